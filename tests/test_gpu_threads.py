"""Two host threads recording on one device (the reference's Device is shared across
threads, crates/eyebrowse-gpu/src/device.rs:20-30; a Recorder belongs to one thread).

Decode and prefill take their scratch space from the device's grow-only workspace. One
thread's launches must never see a buffer that another thread's growth has freed, so
here one thread keeps decoding at a short length while two others grow the workspace
step by step (longer decodes, longer prompts); every output is checked against the
oracle.
"""
import threading

import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_close, note, upload

pytestmark = pytest.mark.gpu


def test_two_threads_share_the_device_workspace(dev):
    note("threads: decode at a fixed length while another thread grows the workspace")
    h, hkv, hd, max_seq = 16, 8, 128, 12288
    sc = float(oracle.default_scale(hd))
    kc, vc = oracle.randn((max_seq, hkv, hd), 40), oracle.randn((max_seq, hkv, hd), 41)
    kt, vt = upload(dev, kc), upload(dev, vc)
    q = oracle.randn((h, hd), 42)
    qt = upload(dev, q)
    short_pos = 700
    grow_pos = [1000, 2000, 3000, 4500, 6000, 8000, 10000, 12000]
    errors = []

    def run(positions, tag):
        try:
            ot = eb.Tensor.empty(dev, (h, hd))
            for pos in positions:
                rec = eb.Recorder(dev)
                eb.attn_decode(rec, qt, kt, vt, ot, h, hkv, pos, hd, max_seq, sc)
                rec.submit()
                got = ot.to_f32().reshape(1, h, hd)
                want = oracle.attn_decode(q, kc, vc, h, hkv, pos, hd, max_seq, sc, threads=8)
                assert_close(got, want.reshape(1, h, hd), what=f"{tag} pos={pos}")
        except Exception as e:  # reported by the main thread
            errors.append(e)

    def grow_prefill():
        # prompts of growing length: each needs a larger pre-split workspace
        try:
            for i, T in enumerate((300, 600, 1200, 2400)):
                pq = oracle.randn((T, h, hd), 50 + i)
                pk, pv = oracle.randn((T, hkv, hd), 60 + i), oracle.randn((T, hkv, hd), 70 + i)
                ot = eb.Tensor.empty(dev, (T, h, hd))
                rec = eb.Recorder(dev)
                eb.attn_prefill(rec, upload(dev, pq), upload(dev, pk), upload(dev, pv), ot, h, hkv,
                                T, hd, sc)
                rec.submit()
                got = ot.to_f32().reshape(T, h, hd)[T - 8:]
                want = oracle.attn_prefill(pq, pk, pv, h, hkv, T, hd, sc, rows=(T - 8, 8),
                                           threads=8)[T - 8:]
                assert_close(got, want, what=f"prefill T={T}")
        except Exception as e:
            errors.append(e)

    a = threading.Thread(target=run, args=([short_pos] * 12, "steady"))
    b = threading.Thread(target=run, args=(grow_pos, "growing"))
    c = threading.Thread(target=grow_prefill)
    c.start()
    a.start()
    b.start()
    for t in (a, b, c):
        t.join(timeout=100)
    assert not any(t.is_alive() for t in (a, b, c)), "a thread did not finish"
    assert not errors, errors[0]
