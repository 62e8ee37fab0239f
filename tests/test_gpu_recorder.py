"""The deferred recorder (eb_recorder_new_deferred): the reference's Recorder semantics
(crates/eyebrowse-gpu/src/recorder.rs:10-35), where nothing recorded runs until submit and
a recorder dropped without a submit discards its work."""
import numpy as np
import pytest

import eyebrowse_amd as eb
import oracle
from tests._gpu import assert_bitwise, note, upload

pytestmark = pytest.mark.gpu

ROWS, DIM, EPS = 4, 256, 1e-6


def _inputs(dev):
    x = oracle.randn((ROWS, DIM), 1)
    w = oracle.randn((DIM,), 2)
    return upload(dev, x), upload(dev, w)


def _immediate(dev, xt, wt):
    out = eb.Tensor.empty(dev, (ROWS, DIM))
    rec = eb.Recorder(dev)
    eb.rmsnorm(rec, xt, wt, out, ROWS, DIM, EPS)
    rec.submit()
    return out.to_f32()


def test_deferred_recorder_runs_at_submit(dev):
    """Recorded work runs at submit and gives the immediate recorder's bits."""
    note("deferred recorder: submit")
    xt, wt = _inputs(dev)
    want = _immediate(dev, xt, wt)
    mid = eb.Tensor.empty(dev, (ROWS, DIM))
    out = upload(dev, np.full((ROWS, DIM), 7.0, np.float32))
    rec = eb.Recorder(dev, deferred=True)
    eb.rmsnorm(rec, xt, wt, mid, ROWS, DIM, EPS)
    eb.rmsnorm(rec, mid, wt, out, ROWS, DIM, EPS)  # a second kernel reading the first's result
    rec.submit()
    twice = eb.Tensor.empty(dev, (ROWS, DIM))
    rec = eb.Recorder(dev)
    eb.rmsnorm(rec, upload(dev, want.reshape(ROWS, DIM)), wt, twice, ROWS, DIM, EPS)
    rec.submit()
    assert_bitwise(out.to_f32(), twice.to_f32(), "deferred two-kernel record vs immediate")


def test_deferred_recorder_dropped_discards_its_work(dev):
    """A deferred recorder released without a submit leaves the output untouched; the
    device records as usual afterwards."""
    note("deferred recorder: drop")
    xt, wt = _inputs(dev)
    fill = np.full((ROWS, DIM), 7.0, np.float32)
    out = upload(dev, fill)
    rec = eb.Recorder(dev, deferred=True)
    eb.rmsnorm(rec, xt, wt, out, ROWS, DIM, EPS)
    rec.release()
    assert_bitwise(out.to_f32(), fill, "output after a dropped deferred recorder")
    rec = eb.Recorder(dev)
    eb.rmsnorm(rec, xt, wt, out, ROWS, DIM, EPS)
    rec.submit()
    assert_bitwise(out.to_f32(), _immediate(dev, xt, wt), "immediate recording afterwards")


def test_deferred_recorder_is_exclusive(dev):
    """While a deferred recorder is open, other recorders, host reads and a second deferred
    recorder on the device are refused; after its submit they work again."""
    note("deferred recorder: exclusive")
    xt, wt = _inputs(dev)
    out = eb.Tensor.empty(dev, (ROWS, DIM))
    rec = eb.Recorder(dev, deferred=True)
    other = eb.Recorder(dev)
    with pytest.raises(eb.EyebrowseError):
        eb.rmsnorm(other, xt, wt, out, ROWS, DIM, EPS)
    with pytest.raises(eb.EyebrowseError):
        out.to_f32()
    with pytest.raises(eb.EyebrowseError):
        eb.Recorder(dev, deferred=True)
    eb.rmsnorm(rec, xt, wt, out, ROWS, DIM, EPS)
    rec.submit()
    other.submit()
    assert_bitwise(out.to_f32(), _immediate(dev, xt, wt), "deferred result")
