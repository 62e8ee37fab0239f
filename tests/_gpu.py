"""Helpers for the GPU parity tests: run one entry point through the C ABI on numpy inputs
and read the result back, plus the tolerances each comparison states."""
import sys

import numpy as np

import eyebrowse_amd as eb
from tests._textbook import rel_l2_f64

# North-star parity bar against the f32 oracle (any MFMA input precision).
NORTH_REL_L2 = 1e-3
NORTH_MAX_ABS = 2e-3
# The prefill kernel multiplies in FP32 on the matrix cores and the decode kernel in FP32
# on the vector ALUs, so both hold a much tighter bar than the north star: only the
# summation order and exp2-vs-expf rounding differ from the oracle.
F32_REL_L2 = 2e-5
F32_MAX_ABS = 1e-4


def note(msg: str) -> None:
    """Name the GPU case about to run (flushed, so a crash still shows it)."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)


def assert_close(got, want, rel=F32_REL_L2, abs_=F32_MAX_ABS, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    r = rel_l2_f64(got, want)
    m = float(np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)))) if got.size else 0
    assert r <= NORTH_REL_L2 and m <= NORTH_MAX_ABS, f"{what}: north-star bar missed rel={r:.3e} max={m:.3e}"
    assert r <= rel and m <= abs_, f"{what}: rel={r:.3e} max={m:.3e}"
    return r, m


def assert_bitwise(got, want, what=""):
    """Bit-for-bit equality of two f32 arrays (reports the mismatch count, not a diff)."""
    g = np.ascontiguousarray(got, np.float32).view(np.uint32).ravel()
    w = np.ascontiguousarray(want, np.float32).view(np.uint32).ravel()
    assert g.size == w.size, f"{what}: {g.size} vs {w.size} elements"
    bad = int(np.count_nonzero(g != w))
    assert bad == 0, f"{what}: {bad} of {g.size} elements differ bitwise"


def upload(dev, a):
    a = np.ascontiguousarray(a, np.float32)
    return eb.Tensor.from_f32(dev, a.shape, a)


def prefill(dev, q, k, v, h, hkv, s, hd, scale):
    qt, kt, vt = upload(dev, q), upload(dev, k), upload(dev, v)
    ot = eb.Tensor.empty(dev, (s, h, hd))
    rec = eb.Recorder(dev)
    eb.attn_prefill(rec, qt, kt, vt, ot, h, hkv, s, hd, scale)
    rec.submit()
    return ot.to_f32().reshape(s, h, hd)


def decode(dev, q, kc, vc, h, hkv, pos, hd, max_seq, scale):
    qt, kt, vt = upload(dev, q), upload(dev, kc), upload(dev, vc)
    ot = eb.Tensor.empty(dev, (h, hd))
    rec = eb.Recorder(dev)
    eb.attn_decode(rec, qt, kt, vt, ot, h, hkv, pos, hd, max_seq, scale)
    rec.submit()
    return ot.to_f32().reshape(h, hd)
