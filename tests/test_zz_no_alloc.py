"""The allocation-free forward entry (pfhip_model_forward_device_noalloc)
against the allocating one (pfhip_model_forward_device), through the C ABI:
the same kernels on the same inputs give bit-identical logits, on two calls
in a row (the second smaller, so a stale larger layout in the shared fixed
scratch would show), and requests beyond the fixed scratch or the RoPE
tables already built fail with an error before any work."""
import numpy as np
import pytest

from textsift_amd import _native, synth
from textsift_amd.config import PF_CONFIG

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_model():
    w = synth.make_model_weights(PF_CONFIG, seed=4242)
    be = _native.Backend(0)
    m = _native.Model(be, PF_CONFIG)
    for name, arr in w.items():
        m.set_weight(name, arr)
    m.finalize()
    yield be, m
    m.close()
    be.close()


def _both(be, m, B, T, seed, masked=False):
    C = PF_CONFIG.num_classes
    ids = be.buffer(synth.token_ids(seed, B * T))
    mask = None
    if masked:
        mk = np.ones(B * T, np.uint8)
        mk[-T // 4:] = 0
        mask = be.buffer(mk)
    la, lb = be.buffer(nbytes=B * T * C * 4), be.buffer(nbytes=B * T * C * 4)
    try:
        m.forward_device(ids, mask, B, T, la)
        m.forward_device_noalloc(ids, mask, B, T, lb)
        a, b = la.read(np.float32), lb.read(np.float32)
    finally:
        for x in (ids, mask, la, lb):
            if x is not None:
                x.release()
    return a, b


def test_noalloc_matches_forward_device_two_calls(full_model):
    be, m = full_model
    for B, T, seed, masked in ((1, 2048, 11, False), (1, 300, 12, True)):
        a, b = _both(be, m, B, T, seed, masked)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (B, T)
    # and again in the other order of sizes on the same shared array
    a, b = _both(be, m, 2, 700, 13)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_rejects_what_does_not_fit(full_model):
    be, m = full_model
    C = PF_CONFIG.num_classes
    ids = be.buffer(np.zeros(8192, np.int32))
    lg = be.buffer(nbytes=8192 * C * 4)
    try:
        with pytest.raises(RuntimeError, match="allocation-free forward"):
            m.forward_device_noalloc(ids, None, 4, 2048, lg)   # scratch of 8192 rows
        with pytest.raises(RuntimeError, match="RoPE tables"):
            m.forward_device_noalloc(ids, None, 1, 2100, lg)   # positions past the tables (2048)
    finally:
        ids.release()
        lg.release()
