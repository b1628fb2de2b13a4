"""The rounding-point emulation (tests/rounding_emulation.py) that the 16-bit tolerances rest on
(no GPU): without rounding it is the oracle's forward, and each operand type's error is what its
precision predicts."""
import numpy as np

import oracle.encoder as E
from laya_cuda import synthetic
import rounding_emulation as R


def _small():
    spec = synthetic.adapter(None, layers=3, width=128, heads=2, intermediate=512, vocab=700, positions=256,
                             max_len=256)
    w = synthetic.weights(spec, seed=5)
    rng = np.random.default_rng(6)
    sequences = [rng.integers(5, 700, n, dtype=np.int32) for n in (200, 57)]
    questions = [(0, [3, 17, 150, 199], 0), (1, [1, 2, 56], 2), (0, [9, 10], 1)]
    return spec, w, sequences, questions


def test_without_rounding_the_emulation_is_the_oracle():
    spec, w, sequences, _ = _small()
    cfg = {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers}
    sw = E.structured(w, cfg)
    for ids in sequences:
        for branch16 in (True, False):
            np.testing.assert_allclose(R.encoder_sequence(ids, sw, cfg, "none", branch16),
                                       E.encoder_sequence(ids, sw, cfg), atol=2e-5)


def test_rounding_helpers_match_numpy_and_bit_patterns():
    x = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -9, -2.5, 3e-8, 65504.0, 1e-3], np.float32)
    np.testing.assert_array_equal(R.f16(x), x.astype(np.float16).astype(np.float32))
    # bf16 keeps 8 significant bits, ties to even: 1 + 2^-8 -> 1, 1 + 3*2^-9 -> 1 + 2^-7.
    np.testing.assert_array_equal(R.bf16(x[:3]), np.array([1.0, 1.0, 1 + 2 ** -7], np.float32))
    assert (R.bf16(x).view(np.uint32) & 0xFFFF == 0).all()


def test_error_grows_with_coarser_operands():
    spec, w, sequences, questions = _small()
    errors = {d: R.logit_error(spec, w, sequences, questions, d)[0] for d in ("none", "float16", "bfloat16")}
    assert errors["none"] < 1e-5
    assert 0 < errors["float16"] < errors["bfloat16"]
    # fp16 has 3 more significand bits than bf16: its error is several times smaller.
    assert errors["bfloat16"] > 3 * errors["float16"]
