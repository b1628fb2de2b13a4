"""laya_predict_static (the entry point that allocates nothing) against laya_predict, through the C
ABI: bit-identical logits and acts on two calls in a row, the second with a smaller request, both
on the same engine and the same device scratch; a shape class whose arena exceeds the scratch is
refused.  The kernels and launch plans are those of laya_predict's forward, so the outputs must
match it bit for bit (its graph replay equals its eager pass bit for bit).
"""
import ctypes as ct

import numpy as np
import pytest

from laya_cuda import _lib, synthetic
from laya_cuda.runtime import Runtime, pack, shape_class

pytestmark = pytest.mark.gpu


def static_predict(rt, sequences, questions, key=None):
    key = key or shape_class(sequences, questions)
    block = pack(sequences, questions, key, rt.adapter.pad, rt.adapter.vocab)
    m, b, k = key
    logits = np.full((b, k), np.nan, np.float32)
    acts = np.full((b, rt.adapter.n_act), np.nan, np.float32)
    metrics = _lib.LayaMetrics()
    rc = _lib.load().laya_predict_static(
        rt._handle, block.ctypes.data_as(ct.POINTER(ct.c_int32)), ct.byref(_lib.LayaShape(m, b, k)),
        logits.ctypes.data_as(ct.POINTER(ct.c_float)), acts.ctypes.data_as(ct.POINTER(ct.c_float)), ct.byref(metrics))
    return rc, logits[:len(questions)], acts[:len(questions)], metrics


def test_static_entry_point_matches_predict_on_consecutive_calls(gpu):
    spec = synthetic.adapter("l512")
    w = synthetic.weights(spec, seed=0)
    rt = Runtime(spec, 0, 4, weights=w)
    try:
        slots_before = len(rt.slots)
        rng = np.random.default_rng(4)
        two_long = [rng.integers(5, spec.vocab, 512, dtype=np.int32), rng.integers(5, spec.vocab, 500, dtype=np.int32)]
        requests = [synthetic.request("l512", seed=1),                                    # 512 rows
                    synthetic.request("l83", seed=1),                                     # smaller: 96 rows
                    (two_long, [(0, [1, 9, 300], 0), (1, [2, 499, 499, 7], 0)])]           # 1,024 rows
        for sequences, questions in requests:
            rc, logits, acts, metrics = static_predict(rt, sequences, questions)
            assert rc == _lib.OK, _lib.error(rt._handle)
            want_logits, want_acts, _ = rt.predict_sequences(sequences, questions)
            np.testing.assert_array_equal(logits, want_logits)
            np.testing.assert_array_equal(acts, want_acts)
            assert metrics.gpu_ms > 0 and not metrics.graph_replay and not metrics.cache_miss
        # The static calls created no shape slot; laya_predict's three did.
        assert slots_before == 0 and len(rt.slots) == 3
        # Again after laya_predict has run: the scratch still holds the previous call's contents.
        sequences, questions = requests[1]
        again = static_predict(rt, sequences, questions)
        np.testing.assert_array_equal(again[1], rt.predict_sequences(sequences, questions)[0])
        # A shape class beyond the scratch is refused before anything runs.
        rc, *_ = static_predict(rt, requests[0][0], requests[0][1], key=(16384, 2, 8))
        assert rc == _lib.EINVAL and "device scratch" in _lib.error(rt._handle)
    finally:
        rt.close()


def test_static_entry_point_matches_predict_for_modernbert(gpu):
    """The ModernBERT variant (RoPE, GeGLU, +-64 windows on local layers, two head layers whose
    buffers are carved from the same scratch): bit-identical to laya_predict on a 700-token pack
    and then a smaller 90-token one."""
    spec = synthetic.modernbert_adapter(layers=3, width=256, heads=4, intermediate=512, vocab=3000, positions=1024,
                                        max_len=1024, head_layers=2)
    w = synthetic.weights(spec, seed=15, random_norms=True)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        rng = np.random.default_rng(16)
        requests = [([rng.integers(5, 3000, 700, dtype=np.int32)], [(0, [3, 88, 650], 1)]),
                    ([rng.integers(5, 3000, 60, dtype=np.int32), rng.integers(5, 3000, 30, dtype=np.int32)],
                     [(0, [1, 2, 59], 0), (1, [5, 29], 2)])]
        for sequences, questions in requests:
            rc, logits, acts, metrics = static_predict(rt, sequences, questions)
            assert rc == _lib.OK, _lib.error(rt._handle)
            want_logits, want_acts, _ = rt.predict_sequences(sequences, questions)
            np.testing.assert_array_equal(logits, want_logits)
            np.testing.assert_array_equal(acts, want_acts)
            assert np.isfinite(logits).all() and metrics.gpu_ms > 0
    finally:
        rt.close()
