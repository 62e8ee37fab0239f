"""kv_write on the GPU: bit-exact against the oracle (crates/eyebrowse-kernels/src/ops.rs:
70-87,150-179), including the reference's own known-answer case (ops.rs:271-292)."""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, note, upload

pytestmark = pytest.mark.gpu


def test_reference_known_answer(dev):
    """ops.rs:271-292: hkv=2, hd=4, max_seq=8, src[i] = i+1 at dst=3; row 0 stays 0."""
    note("kv_write reference case")
    hkv, hd, max_seq = 2, 4, 8
    ct = upload(dev, np.zeros((max_seq, hkv, hd), np.float32))
    src = np.arange(hkv * hd, dtype=np.float32) + 1
    st = upload(dev, src.reshape(1, hkv, hd))
    rec = eb.Recorder(dev)
    eb.kv_write(rec, ct, st, hkv, 1, hd, max_seq, 3)
    rec.submit()
    got = ct.to_f32()
    for head in range(hkv):
        for d in range(hd):
            assert got[(3 * hkv + head) * hd + d] == src[head * hd + d]
    assert got[0] == 0.0
    want = oracle.kv_write(np.zeros(max_seq * hkv * hd, np.float32), src, hkv, 1, hd, 3)
    assert_bitwise(got, want, "kv_write")


@pytest.mark.parametrize("hkv,hd,max_seq,count,dst", [
    (8, 128, 8192, 1, 8191),      # Qwen decode write at the last row
    (8, 128, 8192, 4096, 0),      # Qwen prefill T=4096
    (8, 256, 16384, 1, 16383),    # Gemma decode write
    (8, 256, 4096, 4096, 0),      # Gemma prefill T=4096 (32 MiB)
    (8, 128, 32768, 1, 32767),    # Mistral decode write
    (3, 6, 50, 7, 11),            # ragged: not a multiple of 4 floats (scalar path)
    (1, 4, 9, 0, 9),              # empty write at the end
])
def test_bit_exact_against_oracle(dev, hkv, hd, max_seq, count, dst):
    note(f"kv_write hkv={hkv} hd={hd} max_seq={max_seq} count={count} dst={dst}")
    cache = oracle.randn((max_seq, hkv, hd), 7)
    src = oracle.randn((max(count, 1), hkv, hd), 8)[:count]
    ct = upload(dev, cache)
    st = eb.Tensor.from_f32(dev, (count, hkv, hd), src) if count else eb.Tensor.empty(dev, (0, hkv, hd))
    rec = eb.Recorder(dev)
    eb.kv_write(rec, ct, st, hkv, count, hd, max_seq, dst)
    rec.submit()
    want = oracle.kv_write(cache, src, hkv, count, hd, dst)
    assert_bitwise(ct.to_f32(), want, "kv_write")


def test_special_float_payloads_are_copied_bitwise(dev):
    note("kv_write special values")
    hkv, hd, max_seq = 2, 8, 4
    bits = np.array([0x7FC00001, 0xFFC12345, 0x7F800000, 0xFF800000, 0x80000000, 0x00000001,
                     0x3F800000, 0x7F7FFFFF] * 2, dtype=np.uint32)
    src = bits.view(np.float32).reshape(1, hkv, hd)
    ct = upload(dev, np.zeros((max_seq, hkv, hd), np.float32))
    st = upload(dev, src)
    rec = eb.Recorder(dev)
    eb.kv_write(rec, ct, st, hkv, 1, hd, max_seq, 2)
    rec.submit()
    got = np.frombuffer(ct.read_bytes(), dtype=np.uint32).reshape(max_seq, hkv * hd)
    assert (got[2] == bits).all()
    assert (got[[0, 1, 3]] == 0).all()


def test_out_of_range_write_is_rejected(dev):
    ct = eb.Tensor.empty(dev, (8, 2, 4))
    st = eb.Tensor.empty(dev, (2, 2, 4))
    rec = eb.Recorder(dev)
    with pytest.raises(eb.ShapeMismatch):
        eb.kv_write(rec, ct, st, 2, 2, 4, 8, 7)
    rec.submit()
