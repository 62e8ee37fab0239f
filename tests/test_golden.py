"""CPU: the committed golden vectors still match the oracle bit for bit, and the seeded
input generator still produces the same bytes (tests/golden/gen_golden.py wrote them and
cross-checked each against float64 at the time)."""
import hashlib
import os

import numpy as np

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def test_qwen_t64_prefill_fixture():
    g = load("qwen_t64_prefill.npz")
    T, H, Hkv, hd = int(g["T"]), int(g["H"]), int(g["Hkv"]), int(g["hd"])
    q = oracle.randn((T, H, hd), 1)
    k = oracle.randn((T, Hkv, hd), 2)
    v = oracle.randn((T, Hkv, hd), 3)
    assert (sha(q), sha(k), sha(v)) == (str(g["sha_q"]), str(g["sha_k"]), str(g["sha_v"]))
    o = oracle.attn_prefill(q, k, v, H, Hkv, T, hd, float(g["scale"]))
    assert o.tobytes() == g["o"].tobytes()


def test_qwen_decode_fixture():
    g = load("qwen_decode_small.npz")
    H, Hkv, hd, ms, pos = (int(g[x]) for x in ("H", "Hkv", "hd", "max_seq", "pos"))
    q = oracle.randn((H, hd), 1)
    kc = oracle.randn((ms, Hkv, hd), 2)
    vc = oracle.randn((ms, Hkv, hd), 3)
    assert (sha(q), sha(kc), sha(vc)) == (str(g["sha_q"]), str(g["sha_kc"]), str(g["sha_vc"]))
    o = oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, ms, float(g["scale"]))
    assert o.tobytes() == g["o"].tobytes()


def test_reference_ramp_fixture():
    g = load("reference_ramp_cases.npz")
    o = oracle.attn_prefill(g["prefill_q"], g["prefill_k"], g["prefill_v"], 2, 1, 5, 8)
    assert o.tobytes() == g["prefill_o"].tobytes()
    od = oracle.attn_decode(g["decode_q"], g["decode_k"], g["decode_v"], 4, 2, 5, 8, 16)
    assert od.tobytes() == g["decode_o"].tobytes()
    kvw = oracle.kv_write(np.zeros(64, np.float32), g["kvw_src"], 2, 1, 4, 3)
    assert kvw.tobytes() == g["kvw_cache"].tobytes()


def test_gemma_t32_fixture():
    g = load("gemma_t32_prefill.npz")
    T, H, Hkv, hd = int(g["T"]), int(g["H"]), int(g["Hkv"]), int(g["hd"])
    eps = float(g["eps"])
    q = oracle.randn((T, H, hd), 1)
    k = oracle.randn((T, Hkv, hd), 2)
    v = oracle.randn((T, Hkv, hd), 3)
    assert (sha(q), sha(k), sha(v)) == (str(g["sha_q"]), str(g["sha_k"]), str(g["sha_v"]))
    gq = (1 + 0.1 * oracle.randn((hd,), 4)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 5)).astype(np.float32)
    c, s = oracle.rope_tables(T, hd, float(g["theta"]), rope_angles=int(g["rope_angles"]))
    qr = oracle.rope(oracle.rmsnorm(q, gq, T * H, hd, eps), c, s, T, H, hd)
    kr = oracle.rope(oracle.rmsnorm(k, gk, T * Hkv, hd, eps), c, s, T, Hkv, hd)
    vn = oracle.rmsnorm(v, np.ones(hd, np.float32), T * Hkv, hd, eps)
    assert (sha(qr), sha(kr), sha(vn)) == (str(g["sha_q_rope"]), str(g["sha_k_rope"]),
                                           str(g["sha_v_norm"]))
    o = oracle.attn_prefill(qr, kr, vn, H, Hkv, T, hd, 1.0)
    assert o.tobytes() == g["o"].tobytes()
