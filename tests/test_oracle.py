"""Pins the CPU oracle (oracle/oracle.c) before anything is compared against it.

Each oracle function is checked against something that does not share its code:
float64 textbook attention / RMSNorm / RoPE (tests/_textbook.py), torch's own CPU
scaled_dot_product_attention in float64, closed forms and invariants, and the
reference's own known-answer cases (same ramp inputs and shapes as
crates/eyebrowse-kernels/src/attention.rs:175-233, ops.rs:271-292, rope.rs:92-111,
rmsnorm.rs:72-90, crates/eyebrowse-nn/src/rope.rs:82-104, nn/src/tests.rs:152-177).
A mutation test builds deliberately wrong oracles and shows the checks reject them.
"""
import os
import subprocess
import tempfile
import ctypes

import numpy as np
import pytest

import oracle
from tests._textbook import attention_f64, ramp, rel_l2_f64, rmsnorm_f64, rope_f64

# The oracle is f32 arithmetic; against float64 the residual is f32 rounding only.
F32_VS_F64 = 2e-6


# ---------------------------------------------------------------- attention -------------

@pytest.mark.parametrize("h,hkv,s,hd,scale", [
    (2, 1, 5, 8, None),        # reference prefill known-answer shape (attention.rs:177)
    (4, 2, 9, 16, None),
    (16, 8, 33, 128, None),    # Qwen3 shape, short
    (32, 8, 17, 128, None),    # Mistral GQA ratio 4
    (4, 4, 7, 32, 0.3),        # MHA, explicit scale
    (16, 8, 12, 256, 1.0),     # Gemma hd=256, scale 1.0
])
def test_prefill_matches_f64_textbook(h, hkv, s, hd, scale):
    q = oracle.randn((s, h, hd), 11)
    k = oracle.randn((s, hkv, hd), 12)
    v = oracle.randn((s, hkv, hd), 13)
    sc = oracle.default_scale(hd) if scale is None else scale
    got = oracle.attn_prefill(q, k, v, h, hkv, s, hd, sc)
    want = attention_f64(q, k, v, sc)
    assert rel_l2_f64(got, want) < F32_VS_F64 * (4 if scale == 1.0 else 1)


def test_prefill_matches_torch_sdpa_f64():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as F
    h, hkv, s, hd = 8, 2, 21, 64
    q = oracle.randn((s, h, hd), 1)
    k = oracle.randn((s, hkv, hd), 2)
    v = oracle.randn((s, hkv, hd), 3)
    got = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    tq = torch.from_numpy(q).double().permute(1, 0, 2)[None]
    tk = torch.from_numpy(k).double().permute(1, 0, 2)[None]
    tv = torch.from_numpy(v).double().permute(1, 0, 2)[None]
    ref = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True,
                                         scale=float(oracle.default_scale(hd)), enable_gqa=True)
    want = ref[0].permute(1, 0, 2).numpy()
    assert rel_l2_f64(got, want) < F32_VS_F64


def test_reference_prefill_ramp_case():
    """attention.rs:175-202: h=2, hkv=1, s=5, hd=8 with ramp inputs."""
    h, hkv, s, hd = 2, 1, 5, 8
    q = ramp(h * s * hd, -0.5, 0.011).reshape(s, h, hd)
    k = ramp(hkv * s * hd, -0.3, 0.007).reshape(s, hkv, hd)
    v = ramp(hkv * s * hd, 0.2, 0.013).reshape(s, hkv, hd)
    got = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    assert rel_l2_f64(got, attention_f64(q, k, v, 1 / np.sqrt(8))) < F32_VS_F64


def test_reference_decode_ramp_case():
    """attention.rs:205-233: h=4, hkv=2, hd=8, max_seq=16, pos=5 over ramp caches."""
    h, hkv, hd, max_seq, pos = 4, 2, 8, 16, 5
    q = ramp(h * hd, -0.4, 0.02)
    kc = ramp(hkv * max_seq * hd, -0.2, 0.005)
    vc = ramp(hkv * max_seq * hd, 0.1, 0.009)
    got = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, max_seq)
    k = kc.reshape(max_seq, hkv, hd)[: pos + 1]
    v = vc.reshape(max_seq, hkv, hd)[: pos + 1]
    want = attention_f64(q.reshape(1, h, hd), k, v, 1 / np.sqrt(8), causal=False)[0]
    assert rel_l2_f64(got, want) < F32_VS_F64


@pytest.mark.parametrize("h,hkv,hd,max_seq,pos", [(16, 8, 128, 300, 257), (32, 8, 128, 64, 0),
                                                  (16, 8, 256, 40, 39)])
def test_decode_matches_f64_textbook(h, hkv, hd, max_seq, pos):
    q = oracle.randn((h, hd), 1)
    kc = oracle.randn((max_seq, hkv, hd), 2)
    vc = oracle.randn((max_seq, hkv, hd), 3)
    got = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, max_seq)
    want = attention_f64(q[None], kc[: pos + 1], vc[: pos + 1], 1 / np.sqrt(hd),
                         causal=False)[0]
    assert rel_l2_f64(got, want) < F32_VS_F64


def test_first_row_is_v0_exactly():
    """T=1 (and row 0 of any prefill) attends one key with weight exp(0)/exp(0) = 1."""
    h, hkv, s, hd = 4, 2, 6, 16
    q, k, v = (oracle.randn(sh, sd) for sh, sd in [((s, h, hd), 1), ((s, hkv, hd), 2),
                                                   ((s, hkv, hd), 3)])
    o = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    for hh in range(h):
        np.testing.assert_array_equal(o[0, hh], v[0, hh // (h // hkv)])
    od = oracle.attn_decode(q[0], k, v, h, hkv, 0, hd, s)
    np.testing.assert_array_equal(od, o[0])


def test_scale_zero_is_causal_prefix_mean():
    h, hkv, s, hd = 2, 1, 9, 8
    q, k, v = (oracle.randn(sh, sd) for sh, sd in [((s, h, hd), 1), ((s, hkv, hd), 2),
                                                   ((s, hkv, hd), 3)])
    o = oracle.attn_prefill(q, k, v, h, hkv, s, hd, 0.0)
    want = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, s + 1)[:, None, None]
    np.testing.assert_allclose(o, np.repeat(want, h, axis=1), rtol=0, atol=1e-6)


def test_equal_keys_give_uniform_weights():
    h, hkv, s, hd = 2, 2, 7, 8
    q = oracle.randn((s, h, hd), 1)
    k = np.tile(oracle.randn((1, hkv, hd), 2), (s, 1, 1))
    v = oracle.randn((s, hkv, hd), 3)
    o = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    want = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, s + 1)[:, None, None]
    np.testing.assert_allclose(o, want, rtol=0, atol=2e-6)


def test_gqa_equals_mha_with_repeated_kv():
    h, hkv, s, hd = 8, 2, 11, 16
    q, k, v = (oracle.randn(sh, sd) for sh, sd in [((s, h, hd), 1), ((s, hkv, hd), 2),
                                                   ((s, hkv, hd), 3)])
    a = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    b = oracle.attn_prefill(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), h, h, s, hd)
    np.testing.assert_array_equal(a, b)


def test_decode_equals_prefill_row_bitwise():
    """decode(pos) over the first pos+1 cache rows is prefill row pos: the same
    per-row arithmetic (nn/src/tests.rs:181-244 is this invariant end to end)."""
    h, hkv, s, hd = 16, 8, 40, 128
    q, k, v = (oracle.randn(sh, sd) for sh, sd in [((s, h, hd), 4), ((s, hkv, hd), 5),
                                                   ((s, hkv, hd), 6)])
    o = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    for pos in (0, 1, 17, s - 1):
        od = oracle.attn_decode(q[pos], k, v, h, hkv, pos, hd, s)
        np.testing.assert_array_equal(od, o[pos])


def test_row_subset_matches_full_and_threads_do_not_change_bits():
    h, hkv, s, hd = 16, 8, 50, 128
    q, k, v = (oracle.randn(sh, sd) for sh, sd in [((s, h, hd), 7), ((s, hkv, hd), 8),
                                                   ((s, hkv, hd), 9)])
    full = oracle.attn_prefill(q, k, v, h, hkv, s, hd)
    part = oracle.attn_prefill(q, k, v, h, hkv, s, hd, rows=(20, 13), threads=4)
    np.testing.assert_array_equal(part[20:33], full[20:33])
    assert np.isnan(part[:20]).all() and np.isnan(part[33:]).all()
    par = oracle.attn_prefill(q, k, v, h, hkv, s, hd, threads=4)
    np.testing.assert_array_equal(par, full)


def test_default_scale_is_reference_value():
    for hd in (4, 8, 64, 128, 256):
        assert np.float32(oracle.default_scale(hd)) == np.float32(1.0) / np.sqrt(np.float32(hd))


# ------------------------------------------------------------------ kv_write -------------

def test_kv_write_reference_known_answer():
    """ops.rs:271-292: hkv=2, hd=4, max_seq=8, src[i]=i+1 written at dst=3."""
    hkv, hd, max_seq = 2, 4, 8
    cache = np.zeros(max_seq * hkv * hd, np.float32)
    src = np.arange(hkv * hd, dtype=np.float32) + 1
    got = oracle.kv_write(cache, src, hkv, 1, hd, 3)
    for head in range(hkv):
        for d in range(hd):
            assert got[(3 * hkv + head) * hd + d] == src[head * hd + d]
    assert got[0] == 0.0
    # closed form: a contiguous copy to element offset dst * hkv * hd
    want = cache.copy()
    want[3 * hkv * hd: 4 * hkv * hd] = src
    np.testing.assert_array_equal(got, want)


def test_kv_write_is_contiguous_block_copy():
    hkv, hd, max_seq, count, dst = 8, 128, 64, 13, 40
    cache = oracle.randn((max_seq * hkv * hd,), 1)
    src = oracle.randn((count * hkv * hd,), 2)
    got = oracle.kv_write(cache, src, hkv, count, hd, dst)
    want = cache.copy()
    want[dst * hkv * hd:(dst + count) * hkv * hd] = src
    assert got.tobytes() == want.tobytes()


# ------------------------------------------------------------------ RMSNorm / RoPE -------

def test_rmsnorm_reference_case_and_f64():
    """rmsnorm.rs:72-90 inputs (rows 3, dim 320), checked against float64."""
    rows, dim, eps = 3, 320, 1e-6
    x = (np.arange(rows * dim) % 17).astype(np.float32) * np.float32(0.05) - np.float32(0.4)
    w = np.float32(1.0) + np.arange(dim, dtype=np.float32) * np.float32(0.001)
    got = oracle.rmsnorm(x, w, rows, dim, eps)
    assert rel_l2_f64(got, rmsnorm_f64(x, w, dim, eps)) < 1e-6
    x2 = oracle.randn((40 * 256,), 3)
    w2 = (1 + 0.1 * oracle.randn((256,), 4)).astype(np.float32)
    got2 = oracle.rmsnorm(x2, w2, 40, 256, 1e-6)
    assert rel_l2_f64(got2, rmsnorm_f64(x2, w2, 256, 1e-6)) < 1e-6


def test_rmsnorm_unit_weight_gives_unit_rms():
    x = oracle.randn((10 * 128,), 5) * 3
    y = oracle.rmsnorm(x, np.ones(128, np.float32), 10, 128, 0.0).reshape(10, 128)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-6)


def test_rope_tables_reference_cases():
    """nn/src/tests.rs:152-177 (row 0 is (1, 0); row 3 matches f64) and the partial-table
    test nn/src/rope.rs:82-104 (first rope_angles pairs equal the full table, rest 1/0)."""
    c, s = oracle.rope_tables(8, 4, 10000.0)
    np.testing.assert_array_equal(c[0], 1.0)
    np.testing.assert_array_equal(s[0], 0.0)
    k = np.arange(2)
    ang = 3 * np.power(10000.0, -2.0 * k / 4)
    np.testing.assert_allclose(c[3], np.cos(ang), atol=1e-7)
    np.testing.assert_allclose(s[3], np.sin(ang), atol=1e-7)
    fc, fs = oracle.rope_tables(5, 8, 10000.0)
    pc, ps = oracle.rope_tables(5, 8, 10000.0, rope_angles=2)
    np.testing.assert_array_equal(pc[:, :2], fc[:, :2])
    np.testing.assert_array_equal(ps[:, :2], fs[:, :2])
    np.testing.assert_array_equal(pc[:, 2:], 1.0)
    np.testing.assert_array_equal(ps[:, 2:], 0.0)


def test_gemma_partial_rope_tables():
    """Gemma global layers: rope_angles = floor(0.25 * 256 / 2) = 32, theta 1e6
    (models/gemma4.rs:157-165). Pairs >= 32 are exactly (1, 0)."""
    c, s = oracle.rope_tables(300, 256, 1e6, rope_angles=32)
    p = np.arange(128)
    ang = np.arange(300)[:, None] * np.power(1e6, -2.0 * p / 256)[None, :]
    np.testing.assert_allclose(c[:, :32], np.cos(ang[:, :32]), atol=2e-7)
    np.testing.assert_allclose(s[:, :32], np.sin(ang[:, :32]), atol=2e-7)
    assert (c[:, 32:] == 1.0).all() and (s[:, 32:] == 0.0).all()


def test_rope_reference_case_and_f64():
    """rope.rs:92-111: seq 4, 2 heads, hd 8, theta 1e4, x = i*0.03 - 0.5; plus base_pos."""
    seq, nh, hd = 4, 2, 8
    x = np.arange(seq * nh * hd, dtype=np.float32) * np.float32(0.03) - np.float32(0.5)
    c, s = oracle.rope_tables(16, hd, 10000.0)
    got = oracle.rope(x, c, s, seq, nh, hd)
    assert rel_l2_f64(got, rope_f64(x, seq, nh, hd, 10000.0)) < 1e-6
    got5 = oracle.rope(x, c, s, seq, nh, hd, base_pos=5)
    assert rel_l2_f64(got5, rope_f64(x, seq, nh, hd, 10000.0, base_pos=5)) < 1e-6
    # partial rotary leaves pass-through dims bit-identical
    x2 = oracle.randn((6 * 2 * 256,), 8)
    c2, s2 = oracle.rope_tables(10, 256, 1e6, rope_angles=32)
    y2 = oracle.rope(x2, c2, s2, 6, 2, 256, base_pos=3).reshape(6, 2, 256)
    x2r = x2.reshape(6, 2, 256)
    np.testing.assert_array_equal(y2[..., 32:128], x2r[..., 32:128])
    np.testing.assert_array_equal(y2[..., 160:], x2r[..., 160:])
    assert rel_l2_f64(y2, rope_f64(x2, 6, 2, 256, 1e6, rope_angles=32, base_pos=3)) < 1e-6


def test_rope_preserves_pair_norms():
    x = oracle.randn((5 * 3 * 64,), 9)
    c, s = oracle.rope_tables(5, 64, 10000.0)
    y = oracle.rope(x, c, s, 5, 3, 64).reshape(5, 3, 64).astype(np.float64)
    xr = x.reshape(5, 3, 64).astype(np.float64)
    n_in = xr[..., :32] ** 2 + xr[..., 32:] ** 2
    n_out = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ helpers ----------------

def test_rel_l2_closed_form():
    a = np.array([1.0, 2.0, 3.0], np.float32)
    b = np.array([1.0, 2.0, 5.0], np.float32)
    assert abs(oracle.rel_l2(a, b) - 2.0 / (np.sqrt(30.0) + 1e-12)) < 1e-7
    assert oracle.rel_l2(b, b) == 0.0


def test_prng_range_and_moments():
    x = oracle.prng(1 << 20, 0).astype(np.float64)
    assert x.min() >= -1.0 and x.max() < 1.0
    assert abs(x.mean()) < 3e-3 and abs(x.var() - 1 / 3) < 3e-3
    assert not np.array_equal(oracle.prng(16, 1), oracle.prng(16, 2))
    np.testing.assert_array_equal(oracle.prng(16, 7), oracle.prng(32, 7)[:16])


def _gf2_shift(k):
    """64x64 GF(2) matrix of s -> s << k (k > 0) or s >> -k (k < 0) on the bit vector
    (bit i of s = entry i), in uint64 arithmetic (bits shifted out are dropped)."""
    m = np.zeros((64, 64), np.int64)
    for i in range(64):
        j = i - k
        if 0 <= j < 64:
            m[i, j] = 1
    return m


def _gf2_mul(a, b):
    return (a @ b) % 2


def _gf2_pow(m, n):
    r = np.eye(64, dtype=np.int64)
    while n:
        if n & 1:
            r = _gf2_mul(r, m)
        m = _gf2_mul(m, m)
        n >>= 1
    return r


def _xorshift_matrix():
    """One step of the reference's generator (crates/eyebrowse-nn/src/testutil.rs:34-37:
    s ^= s << 13; s ^= s >> 7; s ^= s << 17) as a linear map over GF(2)^64."""
    eye = np.eye(64, dtype=np.int64)
    step = eye
    for k in (13, -7, 17):
        step = _gf2_mul((eye + _gf2_shift(k)) % 2, step)
    return step


def _bits(s):
    return np.array([(s >> i) & 1 for i in range(64)], np.int64)


def _from_bits(v):
    return sum(int(b) << i for i, b in enumerate(v))


def test_prng_against_gf2_jump_ahead():
    """ebo_prng pinned without iterating its shifts: the state after n steps is M^n s0 for
    the GF(2) matrix M of one xorshift step (matrix powers by repeated squaring), with
    s0 = seed + floor(2^64 / golden ratio) mod 2^64 (the constant derived here from an
    integer square root, not copied), and each output the top 53 bits of the state as a
    double u in [0, 1), then f32(2u - 1). The triple (13, 7, 17) in this order is a
    full-period xorshift: M^(2^64 - 1) = I and M^((2^64 - 1) / p) != I for every prime p of
    2^64 - 1, which a wrong shift or direction would almost surely break."""
    from math import isqrt
    golden = (isqrt(5 << 128) - (1 << 64)) // 2  # floor(2^64 (sqrt 5 - 1) / 2)
    assert golden == 0x9E3779B97F4A7C15
    m = _xorshift_matrix()
    order = (1 << 64) - 1
    assert np.array_equal(_gf2_pow(m, order), np.eye(64, dtype=np.int64))
    for p in (3, 5, 17, 257, 641, 65537, 6700417):
        assert order % p == 0
        assert not np.array_equal(_gf2_pow(m, order // p), np.eye(64, dtype=np.int64)), p

    def expect(seed, n):  # output n (1-based step count n)
        s = _from_bits(_gf2_pow(m, n) @ _bits((seed + golden) % (1 << 64)) % 2)
        u = np.float64(s >> 11) / np.float64(1 << 53)
        return np.float32(u * 2.0 - 1.0)

    for seed in (0, 1, 7, 2 ** 64 - 1, 0x61C8864680B583EB):
        got = oracle.prng(9, seed)
        for i in range(9):
            assert got[i].view(np.uint32) == expect(seed, i + 1).view(np.uint32), (seed, i)
    far = oracle.prng(100001, 3)
    assert far[-1].view(np.uint32) == expect(3, 100001).view(np.uint32)
    # ebo_randn draws its uniforms from the same stream, two per normal (1 - u1, u2):
    z = oracle.randn((3,), 5)
    for i in range(3):
        u = [np.float64(_from_bits(_gf2_pow(m, 2 * i + t) @ _bits((5 + golden) % (1 << 64)) % 2)
                        >> 11) / np.float64(1 << 53) for t in (1, 2)]
        want = np.float32(np.sqrt(-2.0 * np.log(1.0 - u[0])) * np.cos(2.0 * np.pi * u[1]))
        assert abs(int(z[i].view(np.int32)) - int(want.view(np.int32))) <= 1, i


def test_randn_is_standard_normal():
    scipy_stats = pytest.importorskip("scipy.stats")
    z = oracle.randn((1 << 18,), 3).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert scipy_stats.kstest(z, "norm").pvalue > 1e-3
    assert np.isfinite(z).all()


# ------------------------------------------------------ chunked / windowed attention ----

@pytest.mark.parametrize("h,hkv,pos0,rows,hd,window", [
    (4, 2, 0, 9, 16, 0),
    (4, 2, 7, 5, 16, 0),       # continuation chunk
    (16, 8, 40, 9, 128, 0),
    (8, 2, 13, 11, 32, 6),     # window shorter than the chunk
    (4, 1, 0, 20, 8, 4),
    (16, 8, 30, 4, 256, 1000), # window longer than the context: no effect
])
def test_chunk_matches_f64_textbook(h, hkv, pos0, rows, hd, window):
    S = pos0 + rows
    q, k, v = oracle.randn((rows, h, hd), 1), oracle.randn((S, hkv, hd), 2), oracle.randn((S, hkv, hd), 3)
    got = oracle.attn_chunk(q, k, v, h, hkv, pos0, rows, hd, 0.3, window)
    want = attention_f64(q, k, v, 0.3, q_offset=pos0, window=window)
    assert rel_l2_f64(got, want) < F32_VS_F64


def test_chunk_reduces_to_prefill_and_decode_bitwise():
    h, hkv, hd, S = 8, 2, 32, 23
    q, k, v = oracle.randn((S, h, hd), 1), oracle.randn((S, hkv, hd), 2), oracle.randn((S, hkv, hd), 3)
    full = oracle.attn_prefill(q, k, v, h, hkv, S, hd)
    assert np.array_equal(oracle.attn_chunk(q, k, v, h, hkv, 0, S, hd), full)
    # a continuation chunk computes exactly the rows the full prefill computes there
    assert np.array_equal(oracle.attn_chunk(q[10:], k, v, h, hkv, 10, S - 10, hd), full[10:])
    # one row at position p is a decode step at p
    p = 17
    assert np.array_equal(oracle.attn_chunk(q[p:p + 1], k, v, h, hkv, p, 1, hd)[0],
                          oracle.attn_decode(q[p], k, v, h, hkv, p, hd, S))
    # a window covering the whole context changes nothing
    assert np.array_equal(oracle.attn_chunk(q, k, v, h, hkv, 0, S, hd, window=S), full)


def test_window_of_one_returns_the_current_value_row():
    h, hkv, hd, S = 4, 2, 8, 12
    q, k, v = oracle.randn((S, h, hd), 1), oracle.randn((S, hkv, hd), 2), oracle.randn((S, hkv, hd), 3)
    got = oracle.attn_chunk(q, k, v, h, hkv, 0, S, hd, window=1)
    assert np.array_equal(got, np.repeat(v, h // hkv, axis=1))


# ------------------------------------------------------------------ IEEE-half caches ------

def _half_to_f64(bits):
    """binary16 decoded from its fields (sign, 5-bit exponent bias 15, 10-bit fraction)."""
    b = np.asarray(bits, np.int64)
    sign = np.where(b >> 15, -1.0, 1.0)
    e = (b >> 10) & 31
    f = (b & 1023).astype(np.float64)
    val = np.where(e == 0, f * 2.0 ** -24, (1024 + f) * 2.0 ** (e - 25))
    val = np.where(e == 31, np.where(f == 0, np.inf, np.nan), val)
    return sign * val


def test_f16_bits_known_answers():
    """Hand-derived binary16 patterns: ties to even at 1 + 2^-11 and 2^-25, the largest
    finite half, the overflow threshold 65520, signed zero, the smallest subnormal."""
    cases = {1.0: 0x3C00, 1 + 2 ** -11: 0x3C00, 1 + 3 * 2 ** -11: 0x3C02, -2.0: 0xC000,
             65504.0: 0x7BFF, 65519.0: 0x7BFF, 65520.0: 0x7C00, 1e6: 0x7C00, -1e6: 0xFC00,
             -0.0: 0x8000, 2 ** -24: 0x0001, 2 ** -25: 0x0000, 1.5 * 2 ** -25: 0x0001,
             2 ** -14: 0x0400, float("inf"): 0x7C00, float("-inf"): 0xFC00, 0.1: 0x2E66}
    got = oracle.f16_bits(np.array(list(cases), np.float32))
    assert [int(g) for g in got] == list(cases.values())
    nan = oracle.f16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_f16_bits_round_to_nearest_even():
    """Every finite half-range f32 lands on a nearest binary16 (the error is at most half
    the gap to the neighbouring half; on a tie the fraction is even), decoded from the
    bit fields independently of numpy's float16."""
    x = np.concatenate([oracle.randn((20000,), 5) * 3.0,
                        oracle.randn((5000,), 6) * 1e-5,
                        oracle.randn((5000,), 7) * 3e4]).astype(np.float32)
    x = x[np.abs(x) < 65504]
    bits = oracle.f16_bits(x).astype(np.int64)
    val = _half_to_f64(bits)
    assert np.array_equal(bits >> 15, (x < 0).astype(np.int64))   # sign kept, also at -0
    m = bits & 0x7FFF                                         # magnitude pattern
    mag = np.abs(val)
    up = _half_to_f64(m + 1)                                  # next half away from zero
    dn = np.where(m > 0, _half_to_f64(np.maximum(m - 1, 0)), -_half_to_f64(np.ones_like(m)))
    ax = np.abs(x.astype(np.float64))
    assert np.all(ax - mag <= (up - mag) / 2) and np.all(mag - ax <= (mag - dn) / 2)
    tie = ((ax - mag == (up - mag) / 2) | (mag - ax == (mag - dn) / 2)) & (ax != mag)
    assert np.all((bits[tie] & 1) == 0)
    assert np.array_equal(oracle.f16_values(bits.astype(np.uint16)), val.astype(np.float32))


def test_kv_write_f16_places_rounded_rows():
    hkv, hd, count, start, max_seq = 2, 8, 3, 4, 9
    cache = np.arange(max_seq * hkv * hd, dtype=np.uint16)
    src = oracle.randn((count, hkv, hd), 8)
    got = oracle.kv_write_f16(cache, src, hkv, count, hd, start)
    a, b = start * hkv * hd, (start + count) * hkv * hd
    assert np.array_equal(got[:a], cache[:a]) and np.array_equal(got[b:], cache[b:])
    assert np.array_equal(_half_to_f64(got[a:b]),
                          _half_to_f64(oracle.f16_bits(src.ravel())))
    assert np.max(np.abs(oracle.f16_values(got[a:b]) - src.ravel())) <= 2.0 ** -11 * 4


def _e4m3_to_f64(bits):
    """OCP E4M3 decoded from its fields (sign, 4-bit exponent bias 7, 3-bit fraction; no
    infinities, S.1111.111 NaN)."""
    b = np.asarray(bits, np.int64)
    sign = np.where(b >> 7, -1.0, 1.0)
    e = (b >> 3) & 15
    f = (b & 7).astype(np.float64)
    val = np.where(e == 0, f * 2.0 ** -9, (8 + f) * 2.0 ** (e - 10))
    val = np.where((e == 15) & (f == 7), np.nan, val)
    return sign * val


def test_f8_decode_every_pattern():
    """All 256 patterns against the bit fields and against torch's float8_e4m3fn (an
    independent implementation of the format): 448 largest, 2^-9 smallest subnormal,
    2^-6 smallest normal, 0x7F / 0xFF NaN, signed zeros."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.f8_values(codes)
    want = _e4m3_to_f64(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and list(np.flatnonzero(nan)) == [0x7F, 0xFF]
    assert np.array_equal(got[~nan].astype(np.float64), want[~nan])
    assert np.array_equal(np.signbit(got[~nan]), codes[~nan] >= 0x80)
    tch = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(got[~nan].view(np.uint32), tch[~nan].view(np.uint32))
    pos = got[:0x7F]
    assert np.all(np.diff(pos) > 0) and pos[-1] == 448.0
    assert pos[1] == 2.0 ** -9 and pos[8] == 2.0 ** -6


def test_f8_bits_known_answers():
    """Hand-derived patterns: ties to the even fraction (1 + 2^-4 -> 1, 1 + 3 * 2^-4 -> 1.25,
    464 -> 448, 1.5 * 2^-9 -> 2^-8), saturation of finite values at and beyond 448, inf and
    NaN to NaN, signed zero, subnormal steps of 2^-9."""
    cases = [(1.0, 0x38), (1 + 2 ** -4, 0x38), (1 + 3 * 2 ** -4, 0x3A), (-2.0, 0xC0),
             (448.0, 0x7E), (463.9, 0x7E), (464.0, 0x7E), (500.0, 0x7E), (3e38, 0x7E),
             (-1e6, 0xFE), (0.0, 0x00), (-0.0, 0x80), (2 ** -9, 0x01), (2 ** -10, 0x00),
             (1.5 * 2 ** -9, 0x02), (2.5 * 2 ** -9, 0x02), (7.5 * 2 ** -9, 0x08),
             (2 ** -6, 0x08), (0.1, 0x1D), (240.0, 0x77), (416.0, 0x7D)]
    got = oracle.f8_bits(np.array([c[0] for c in cases], np.float32))
    assert [int(g) for g in got] == [c[1] for c in cases]
    special = oracle.f8_bits(np.array([np.inf, -np.inf, np.nan, -np.nan], np.float32))
    assert [int(g) for g in special] == [0x7F, 0xFF, 0x7F, 0xFF]


def test_f8_bits_nearest_even_and_torch():
    """Random values over the whole range and every midpoint between neighbouring values
    (with the f32 neighbours either side): the result is a nearest E4M3 value (ties to the
    even fraction), and below 448 it equals torch's float8_e4m3fn conversion bit for bit."""
    import torch
    x = np.concatenate([oracle.randn((40000,), 11) * s for s in (2e-3, 0.05, 1.0, 20.0, 150.0)])
    fin = _e4m3_to_f64(np.arange(0x7F))  # the finite non-negative values, ascending
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.nextafter(mids, np.float32(0)),
                        np.nextafter(mids, np.float32(1e9))]).astype(np.float32)
    bits = oracle.f8_bits(x).astype(np.int64)
    assert np.array_equal(bits >> 7, np.signbit(x).astype(np.int64))
    ax = np.abs(x.astype(np.float64))
    mag = np.abs(_e4m3_to_f64(bits))
    inr = ax < 448
    d = np.abs(ax[:, None] - fin[None, :])[inr]   # brute force over every finite value
    best = d.min(axis=1)
    assert np.all(np.abs(ax[inr] - mag[inr]) == best)
    tie = (d == best[:, None]).sum(axis=1) > 1
    assert np.all((bits[inr][tie] & 1) == 0)
    assert np.all(mag[~inr] == 448.0)
    y = x[inr]
    tch = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.f8_bits(y), tch)


def test_kv_write_f8_places_rounded_rows():
    hkv, hd, count, start, max_seq = 2, 16, 3, 4, 9
    cache = (np.arange(max_seq * hkv * hd) % 251).astype(np.uint8)
    src = oracle.randn((count, hkv, hd), 8)
    got = oracle.kv_write_f8(cache, src, hkv, count, hd, start)
    a, b = start * hkv * hd, (start + count) * hkv * hd
    assert np.array_equal(got[:a], cache[:a]) and np.array_equal(got[b:], cache[b:])
    assert np.array_equal(got[a:b], oracle.f8_bits(src.ravel()))
    err = np.abs(oracle.f8_values(got[a:b]) - src.ravel())
    assert np.all(err <= np.maximum(np.abs(src.ravel()) * 2.0 ** -4, 2.0 ** -10))


# ------------------------------------------------------------------ linear_f16w / argmax --

def test_f16_decode_matches_numpy_for_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    lib = oracle._load()
    got = np.array([lib.ebo_f16_to_f32(int(b)) for b in bits], np.float32)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_pack_f16_reference_layout():
    """tensor.rs:7-23: low half first, odd tail zero-padded."""
    assert [int(v) for v in oracle.pack_f16(np.array([1.0, -2.0, 0.5], np.float32))] == \
        [0xC0003C00, 0x00003800]


def test_linear_reference_ramp_case():
    """matmul.rs:255-272: m=5, in=33, out=7 ramps; the reference asserts rel-L2 < 2e-3
    against its CPU linear on f16-rounded weights. Here against float64."""
    m, in_f, out_f = 5, 33, 7
    x = (np.arange(m * in_f) * 0.01 - 0.2).astype(np.float32).reshape(m, in_f)
    w = (np.arange(out_f * in_f) * 0.005 - 0.3).astype(np.float32).reshape(out_f, in_f)
    wb = oracle.f16_bits(w)
    got = oracle.linear_f16w(x, wb, m, in_f, out_f)
    want = x.astype(np.float64) @ oracle.f16_values(wb).reshape(out_f, in_f).astype(np.float64).T
    assert rel_l2_f64(got, want) < 1e-6


@pytest.mark.parametrize("m,in_f,out_f", [(1, 1024, 64), (7, 96, 130), (33, 256, 48),
                                          (2, 4096, 16)])
def test_linear_matches_f64(m, in_f, out_f):
    x = oracle.randn((m, in_f), 1)
    wb = oracle.f16_bits(oracle.randn((out_f, in_f), 2) * 0.05)
    got = oracle.linear_f16w(x, wb, m, in_f, out_f, threads=8)
    w64 = oracle.f16_values(wb).reshape(out_f, in_f).astype(np.float64)
    want = x.astype(np.float64) @ w64.T
    # sequential f32 accumulation: error within in_f unit roundoffs of the row's scale
    bound = in_f * 2.0 ** -24
    assert rel_l2_f64(got, want) < bound
    assert np.max(np.abs(got - want)) <= bound * np.max(np.abs(want))


def test_linear_identity_and_single_column_exact():
    """w = I gives x back exactly; a one-hot row picks one column of x exactly."""
    n = 40
    x = oracle.randn((3, n), 3)
    y = oracle.linear_f16w(x, oracle.f16_bits(np.eye(n, dtype=np.float32)), 3, n, n)
    assert np.array_equal(y, x)
    w = np.zeros((2, n), np.float32)
    w[0, 5] = 1.0
    w[1, 7] = -2.0
    y = oracle.linear_f16w(x, oracle.f16_bits(w), 3, n, 2)
    assert np.array_equal(y[:, 0], x[:, 5]) and np.array_equal(y[:, 1], -2 * x[:, 7])


def _bitrev8(t):
    return int(f"{t:08b}"[::-1], 2)


def _argmax_rule(x):
    """The reference's argmax in closed form: among the indices holding the largest value
    above -3e38 (NaN excluded), the one whose lane i mod 256 comes first in bit-reversed
    order, then the smallest i; 0 if there is none. (Each lane keeps its first maximum.
    In the tree, lane t sits at position t mod s before stride s; two lanes first meet at
    the stride of their lowest differing bit, and the one with that bit clear is on the
    left, which keeps ties.)"""
    x = np.asarray(x, np.float32)
    ok = (x > np.float32(-3e38)) & ~np.isnan(x)
    if not ok.any():
        return 0
    m = x[ok].max()
    idx = np.nonzero(ok & (x == m))[0]
    return int(min(idx, key=lambda i: (_bitrev8(i % 256), i)))


def signed_zero_cases():
    """Vectors whose maximum is zero held with both signs: two-element pairs, a short
    all-nonpositive vector, and vocabularies of one and of several 4096-entry slices with
    the zeros of both signs spread over lanes and slices."""
    out = [np.array([-0.0, 0.0], np.float32), np.array([0.0, -0.0], np.float32)]
    z = np.full(8, -1.0, np.float32)
    z[1], z[2] = 0.0, -0.0
    out.append(z)
    for n, seed in ((4096, 1), (151936, 2), (9001, 3)):
        v = -np.abs(oracle.randn((n,), 300 + seed)) - np.float32(0.5)
        rng = np.random.default_rng(seed)
        pos = rng.choice(n, 40, replace=False)
        v[pos[:20]] = 0.0
        v[pos[20:]] = -0.0
        out.append(v.astype(np.float32))
    return out


def test_argmax_reference_case_and_ties():
    """sampling.rs:62-80 (vocab 1000, sin ramp, unique max at 731); ties across lanes go
    by the tree (index 256, lane 0, beats index 1; lane 116 beats lane 44); NaN and -inf
    never win."""
    v = np.sin(np.arange(1000, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    v[731] = 5.0
    assert oracle.argmax(v) == 731
    assert oracle.argmax(np.array([1, 7, 3, 7], np.float32)) == 1
    t = np.zeros(600, np.float32)
    t[1] = t[256] = t[513] = 2.0
    assert oracle.argmax(t) == 256
    t = np.zeros(300, np.float32)
    t[44] = t[116] = 1.0
    assert oracle.argmax(t) == 116
    assert oracle.argmax(np.array([np.nan, 2, np.nan, 1], np.float32)) == 1
    assert oracle.argmax(np.full(5, -np.inf, np.float32)) == 0
    assert oracle.argmax(np.array([-3.1e38, -3.3e38], np.float32)) == 0
    # -0.0 and +0.0 tie under the strict `>`: lane order decides, never the sign bit
    # (lane 2 precedes lane 1 in bit-reversed order, whichever holds -0.0).
    for case in signed_zero_cases():
        assert oracle.argmax(case) == _argmax_rule(case), case[:8]
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 0
    assert oracle.argmax(np.array([0.0, -0.0], np.float32)) == 0
    z = np.full(8, -1.0, np.float32)
    z[1], z[2] = 0.0, -0.0
    assert oracle.argmax(z) == 2
    z[1], z[2] = -0.0, 0.0
    assert oracle.argmax(z) == 2
    for seed in range(20):
        r = oracle.randn((3000,), seed)
        r = np.round(r * 2) / 2  # many ties
        if seed % 3 == 0:
            r[seed::7] = np.nan
        assert oracle.argmax(r) == _argmax_rule(r)
    r = oracle.randn((151936,), 99)
    assert oracle.argmax(r) == int(np.argmax(r))


def _planted(plant, td):
    src = os.path.join(os.path.dirname(oracle.__file__), "oracle.c")
    so = os.path.join(td, f"planted{plant}.so")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-fopenmp",
                    f"-DEBO_PLANT={plant}", "-o", so, src, "-lm"], check=True)
    return ctypes.CDLL(so)


def test_linear_check_rejects_transposed_weight():
    """EBO_PLANT=5 reads the weight as [in, out]; the float64 check above rejects it."""
    with tempfile.TemporaryDirectory() as td:
        lib = _planted(5, td)
        f32p = ctypes.POINTER(ctypes.c_float)
        lib.ebo_linear_f16w.argtypes = [f32p, ctypes.POINTER(ctypes.c_uint16), f32p,
                                        ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                        ctypes.c_int]
        m, in_f, out_f = 3, 24, 24
        x = oracle.randn((m, in_f), 1)
        wb = oracle.f16_bits(oracle.randn((out_f, in_f), 2))
        y = np.empty((m, out_f), np.float32)
        lib.ebo_linear_f16w(x.ctypes.data_as(f32p),
                            wb.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                            y.ctypes.data_as(f32p), m, in_f, out_f, 1)
        want = x.astype(np.float64) @ oracle.f16_values(wb).reshape(out_f, in_f).T
        assert rel_l2_f64(y, want) > 1e-3


@pytest.mark.parametrize("plant", [1, 2, 3, 4])
def test_checks_reject_planted_oracle_mistakes(plant):
    """Build the oracle with a planted mistake (GQA grouping, causal diagonal, scale,
    V read from K) and show the float64 textbook check above rejects it."""
    src = os.path.join(os.path.dirname(oracle.__file__), "oracle.c")
    with tempfile.TemporaryDirectory() as td:
        so = os.path.join(td, f"planted{plant}.so")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-fopenmp",
                        f"-DEBO_PLANT={plant}", "-o", so, src, "-lm"], check=True)
        lib = ctypes.CDLL(so)
        f32p = ctypes.POINTER(ctypes.c_float)
        sz = ctypes.c_size_t
        lib.ebo_attn_prefill_rows.argtypes = [f32p, f32p, f32p, f32p, sz, sz, sz, sz,
                                              ctypes.c_float, sz, sz, ctypes.c_int]
        h, hkv, s, hd = 4, 2, 9, 16
        q, k, v = (oracle.randn(sh, sd) for sh, sd in [((s, h, hd), 1), ((s, hkv, hd), 2),
                                                       ((s, hkv, hd), 3)])
        o = np.empty((s, h, hd), np.float32)
        sc = 0.25
        p = lambda a: a.ctypes.data_as(f32p)  # noqa: E731
        lib.ebo_attn_prefill_rows(p(q), p(k), p(v), p(o), h, hkv, s, hd, sc, 0, s, 1)
        assert rel_l2_f64(o, attention_f64(q, k, v, sc)) > 1e-3
