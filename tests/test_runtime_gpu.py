"""End-to-end parity of the HIP encoder path against the CPU oracle, and slot/graph lifecycle.

Bar: bit-exact gathers (kernel tests), max |logit - oracle| <= 1e-3 with fp32
accumulation and identical argmax decisions; graph replays bit-equal to eager passes.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle.encoder as E
from laya_cuda import synthetic
from laya_cuda.runtime import Runtime

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
LOGIT_ATOL = 1e-3
# Documented near-ties of the ragged 32-request workload: question 40's two best options are
# 1.2e-5 apart in the oracle, well inside the logit error bound, so either order is a correct
# reading of the same scores.  No other question may change its decision.
RAGGED32_TIES = {40: 1.2e-5}


def _cfg(spec):
    return {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers}


def oracle_logits(spec, w, sequences, questions):
    logits, acts, _ = E.forward(sequences, questions, E.structured(w, _cfg(spec)), _cfg(spec))
    return logits, acts


def decisions(got_logits, want_logits, worst, known_ties=()):
    """Flipped decisions [(question, oracle gap)]: questions whose GPU argmax differs from the
    oracle's.  Every flip must be a documented near-tie, listed in ``known_ties`` by question
    index, whose oracle gap is within 2*worst (two logits each off by at most ``worst`` can swap
    order only then).  Exact ties (duplicate option positions) give bit-identical logits on both
    sides and break to the first index identically, so they never flip."""
    flips = []
    for q, want in enumerate(want_logits):
        mine, theirs = int(np.argmax(got_logits[q, :len(want)])), int(np.argmax(want))
        if mine != theirs:
            flips.append((q, float(want[theirs] - want[mine])))
    for q, gap in flips:
        assert q in known_ties and gap <= 2 * worst, f"question {q}: decision differs, oracle gap {gap:.3e}"
    return flips


def compare(got_logits, got_acts, want_logits, want_acts, atol=LOGIT_ATOL, acts_atol=None, known_ties=(), label=""):
    worst = max(float(np.abs(got_logits[q, :len(w)] - w).max()) for q, w in enumerate(want_logits))
    flips = decisions(got_logits, want_logits, worst, known_ties)
    print(f"{label}: {len(want_logits) - len(flips)}/{len(want_logits)} decisions equal, flips {flips}, "
          f"max |logit error| {worst:.3e}", flush=True)
    assert worst <= atol, f"max |logit error| {worst:.3e} > {atol}"
    np.testing.assert_allclose(got_acts, want_acts, atol=atol if acts_atol is None else acts_atol)
    return worst


def test_small_encoder_matches_golden_and_oracle(gpu):
    spec = synthetic.adapter(None, layers=2, width=128, heads=2, intermediate=512, vocab=1000, positions=64,
                             max_len=64)
    g = np.load(GOLDEN / "bert_small.npz")
    w = synthetic.weights(spec, seed=int(g["seed"]), random_norms=True, std=float(g["std"]))
    sequences = [g[f"ids{s}"] for s in range(int(g["n_seq"]))]
    questions = [(int(g[f"q{q}_seq"]), list(g[f"q{q}_markers"]), int(g[f"q{q}_kind"])) for q in range(int(g["n_q"]))]
    rt = Runtime(spec, 0, 4, weights=w)
    try:
        logits, acts, metrics = rt.predict_sequences(sequences, questions)
        golden = [g[f"q{q}_logits"] for q in range(len(questions))]
        compare(logits, acts, golden, np.stack([g[f"q{q}_acts"] for q in range(len(questions))]), atol=5e-3,
                label="bert small vs transformers golden")
        want, want_acts = oracle_logits(spec, w, sequences, questions)
        compare(logits, acts, want, want_acts, atol=5e-3, label="bert small vs oracle")
        assert metrics["cache_miss"] and metrics["graph_capture"] and metrics["graph_replay"]
    finally:
        rt.close()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("name", ["l83", "l512"])
def test_workload_matches_oracle(gpu, name, dtype):
    """fp16 operands meet the 1e-3 logit bound with room (CPU emulation of this path's rounding
    points: 1.8e-4 at l512).  bf16 operands cannot: rounding only the fp32 weights to bf16 already
    moves the l512 logits by 1.1e-3 in that emulation, and all of this path's bf16 rounding points
    together by 1.39e-3, so bf16 is held to 2e-3 and identical decisions."""
    spec = synthetic.adapter(name, mfma_dtype=dtype)
    w = synthetic.weights(spec, seed=0)
    sequences, questions = synthetic.request(name, seed=1)
    want, want_acts = oracle_logits(spec, w, sequences, questions)
    rt = Runtime(spec, 0, 4, weights=w)
    try:
        logits, acts, _ = rt.predict_sequences(sequences, questions)
        compare(logits, acts, want, want_acts, atol=LOGIT_ATOL if dtype == "float16" else 2e-3, label=f"{name} {dtype}")
        eager = rt.predict_sequences(sequences, questions, capture=False)
        np.testing.assert_array_equal(eager[0], logits)
        np.testing.assert_array_equal(eager[1], acts)
    finally:
        rt.close()


def test_ragged_batch_matches_oracle(gpu):
    spec = synthetic.adapter("ragged32")
    w = synthetic.weights(spec, seed=0)
    sequences, questions = synthetic.request("ragged32", seed=1)
    want, want_acts = oracle_logits(spec, w, sequences, questions)
    rt = Runtime(spec, 0, 4, weights=w)
    try:
        logits, acts, metrics = rt.predict_sequences(sequences, questions)
        compare(logits, acts, want, want_acts, known_ties=RAGGED32_TIES, label=f"ragged32 {metrics['shape']}")
    finally:
        rt.close()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_batched_encoder_matches_oracle(gpu, dtype):
    """A batched slot (more than 4,096 packed rows): the large-tile GEMM pipeline and the 16-bit
    out/down projection rows with their bias added before rounding, as the reference's branch
    buffer.  Tolerances as for the batch-1 workloads (fp16 1e-3, bf16 2e-3)."""
    spec = synthetic.adapter(None, layers=2, width=256, heads=4, intermediate=1024, vocab=3000, positions=1024,
                             max_len=1024, mfma_dtype=dtype)
    w = synthetic.weights(spec, seed=3)
    rng = np.random.default_rng(5)
    lengths = rng.integers(300, 1000, 9)
    sequences = [rng.integers(5, 3000, int(n), dtype=np.int32) for n in lengths]
    questions = [(i, sorted(rng.choice(np.arange(1, int(n)), 5, replace=False).tolist()), i % 3)
                 for i, n in enumerate(lengths)]
    want, want_acts = oracle_logits(spec, w, sequences, questions)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        logits, acts, metrics = rt.predict_sequences(sequences, questions)
        assert metrics["shape"][0] >= 4096, metrics["shape"]
        compare(logits, acts, want, want_acts, atol=LOGIT_ATOL if dtype == "float16" else 2e-3,
                label=f"batched {dtype} rows {metrics['shape'][0]}")
    finally:
        rt.close()


def _large_batch(seed=23):
    spec = synthetic.adapter(None, layers=2, width=256, heads=4, intermediate=1024, vocab=3000, positions=1024,
                             max_len=1024)
    w = synthetic.weights(spec, seed=seed)
    rng = np.random.default_rng(seed + 1)
    lengths = rng.integers(700, 1000, 16)
    sequences = [rng.integers(5, 3000, int(n), dtype=np.int32) for n in lengths]
    questions = [(i, sorted(rng.choice(np.arange(1, int(n)), 4, replace=False).tolist()), i % 3)
                 for i, n in enumerate(lengths)]
    return spec, w, sequences, questions


_CHILD = """
import sys
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2], sys.argv[3]]
from test_runtime_gpu import _large_batch
from laya_cuda.runtime import Runtime
spec, w, sequences, questions = _large_batch()
rt = Runtime(spec, 0, 1, weights=w)
try:
    logits, acts, _ = rt.predict_sequences(sequences, questions)
finally:
    rt.close()
np.savez(sys.argv[4], logits=logits, acts=acts)
"""


def test_large_batched_slot_is_reproducible_across_processes(gpu, tmp_path):
    """A batched slot past 12,288 packed rows (every projection on this library's MFMA tiles, the
    out/down projections as 16-bit rows with the bias before the rounding): fp16 logits within
    1e-3 of the oracle, the graph replay equal to the eager forward bit for bit, and a second
    process computing the same request bit for bit: every launch shape is a pure function of the
    slot's shape and the device, never chosen by timing."""
    import subprocess
    import sys
    spec, w, sequences, questions = _large_batch()
    want, want_acts = oracle_logits(spec, w, sequences, questions)
    rt = Runtime(spec, 0, 1, weights=w)
    try:
        logits, acts, metrics = rt.predict_sequences(sequences, questions)
        assert metrics["shape"][0] >= 12288 and metrics["graph_replay"], metrics["shape"]
        eager = rt.predict_sequences(sequences, questions, capture=False)
        np.testing.assert_array_equal(eager[0], logits)
        np.testing.assert_array_equal(eager[1], acts)
        compare(logits, acts, want, want_acts, label=f"batched slot rows {metrics['shape'][0]}")
    finally:
        rt.close()
    here = Path(__file__).resolve().parent
    out = tmp_path / "child.npz"
    print("starting the second process", flush=True)
    subprocess.run([sys.executable, "-c", _CHILD, str(here), str(here.parent), str(here.parent / "laya-cuda_amd"),
                    str(out)], check=True, timeout=100)
    other = np.load(out)
    np.testing.assert_array_equal(other["logits"], logits)
    np.testing.assert_array_equal(other["acts"], acts)


@pytest.mark.parametrize("hidden", [1024, 16384])
def test_wide_act_head_matches_oracle(gpu, hidden):
    """Act heads wider than the reference's 256 (the C ABI takes any multiple of 64 up to 16,384):
    the head tail's outputs past its 512 threads and its unprefetched act_head.2 rows (1,024), and
    a tail LDS past the default 64 KB (16,384 hidden values plus the logits), against the oracle."""
    spec = synthetic.adapter(None, layers=2, width=64, heads=1, intermediate=256, vocab=500, positions=128,
                             max_len=128)
    spec.act_hidden = hidden
    w = synthetic.weights(spec, seed=29)
    rng = np.random.default_rng(30)
    lengths = [70, 33]
    sequences = [rng.integers(5, 500, n, dtype=np.int32) for n in lengths]
    questions = [(0, [3, 9, 20, 41, 60], 0), (1, [2, 30], 2), (0, [7], 1)]
    want, want_acts = oracle_logits(spec, w, sequences, questions)
    rt = Runtime(spec, 0, 1, weights=w)
    try:
        logits, acts, _ = rt.predict_sequences(sequences, questions)
        compare(logits, acts, want, want_acts, label=f"act head {hidden}")
    finally:
        rt.close()


def test_reference_items_each_question_its_own_row(gpu):
    """Runtime.predict(items) packs every question as its own sequence (runtime.py:52-68)."""
    spec = synthetic.adapter(None, layers=2, width=128, heads=2, intermediate=512, vocab=1000, positions=64,
                             max_len=64)
    w = synthetic.weights(spec, seed=7)
    rng = np.random.default_rng(8)
    items = [(list(rng.integers(5, 1000, n)), sorted(rng.choice(np.arange(1, n), c, replace=False).tolist()), kind)
             for n, c, kind in [(20, 3, 0), (50, 2, 1), (9, 1, 2)]]
    rt = Runtime(spec, 0, 4, weights=w)
    try:
        logits, acts, metrics = rt.predict(items)
        assert metrics["shape"] == (128, 4, 8)
        want, want_acts = oracle_logits(spec, w, [i[0] for i in items], [(q, i[1], i[2]) for q, i in enumerate(items)])
        compare(logits, acts, want, want_acts, label="reference items")
    finally:
        rt.close()


def test_slot_lifecycle_graph_replay_and_eviction(gpu):
    """tests/test_runtime.py:13-53 of the reference, on a synthetic checkpoint."""
    spec = synthetic.adapter(None, layers=2, width=128, heads=2, intermediate=512, vocab=1000, positions=64,
                             max_len=64)
    w = synthetic.weights(spec, seed=11)
    rng = np.random.default_rng(12)
    short = [(list(rng.integers(5, 1000, 12)), [1, 2], 0)]
    long = [(list(rng.integers(5, 1000, 60)), [5, 9, 30], 0)]
    other = [(list(rng.integers(5, 1000, 12)), [3, 4], 0)]
    rt = Runtime(spec, 0, 1, weights=w)
    try:
        first = rt.predict(short)
        assert first[2]["cache_miss"] and first[2]["graph_capture"] and first[2]["graph_replay"]
        again = rt.predict(short)
        assert not again[2]["cache_miss"] and not again[2]["graph_capture"] and again[2]["graph_replay"]
        np.testing.assert_array_equal(first[0], again[0])
        raw = rt.predict(short, capture=False)
        np.testing.assert_array_equal(raw[0], first[0])
        np.testing.assert_array_equal(raw[1], first[1])
        # reusing one graph must upload new contents, not return the previous answer
        changed = rt.predict(other)
        assert not np.array_equal(changed[0], first[0])
        np.testing.assert_array_equal(rt.predict(other, capture=False)[0], changed[0])
        rt.predict(long)
        assert len(rt.slots) == 1
        back = rt.predict(short)
        assert back[2]["cache_miss"] and back[2]["graph_capture"]
        np.testing.assert_array_equal(back[0], first[0])
        assert rt.pool.used_bytes() > 0
        np.testing.assert_array_equal(rt.weights["act_head.2.bias"].get(), w["act_head.2.bias"])
    finally:
        rt.close()
    assert rt.pool.used_bytes() == 0
    with pytest.raises(RuntimeError, match="closed"):
        rt.predict(short)


def test_changed_weights_change_the_answer(gpu):
    """tests/test_custom_models.py:14-57: zero weights, the act probability follows the bias."""
    spec = synthetic.adapter(None, layers=1, width=64, heads=1, intermediate=256, vocab=100, positions=64,
                             max_len=64)
    weights = {name: np.zeros(shape, np.float32) for name, shape in spec.weight_shapes().items()}
    for name in weights:
        if "norm" in name and name.endswith("weight") or name == "scorer.0.weight":
            weights[name][:] = 1
    probs = []
    for bias in ([-4, 4], [4, -4]):
        weights["act_head.2.bias"] = np.array(bias, np.float32)
        rt = Runtime(spec, 0, 2, weights=weights)
        try:
            _, acts, _ = rt.predict([([1, 2, 3, 4], [1, 2], 0)])
            e = np.exp(acts[0] - acts[0].max())
            probs.append(e[0] / e.sum())
        finally:
            rt.close()
    assert probs[0] < .001 and probs[1] > .999
    weights["act_head.2.bias"] = np.zeros(3, np.float32)
    with pytest.raises(ValueError, match="Incompatible tensor shape"):
        Runtime(spec, 0, 2, weights=weights)


# ---------------- ModernBERT variant: the reference's executor for real Laya checkpoints ----------------

def _modern_oracle(spec, w, items):
    import oracle.modernbert as MB
    logits, acts, _ = MB.forward(items, MB.structured(w, MB.config(spec)), MB.config(spec))
    return logits, acts


def _modern_small(dtype):
    return synthetic.modernbert_adapter(layers=4, width=128, heads=2, intermediate=256, vocab=1000, positions=512,
                                        max_len=512, head_layers=2, mfma_dtype=dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_modernbert_small_matches_golden_and_oracle(gpu, dtype):
    """4 layers (global 0 and 3, local 1 and 2 with the +-64 window), RoPE, GeGLU, two head layers;
    fixtures from transformers' ModernBertModel and torch's TransformerEncoderLayer.

    The fixture's weights (std 0.15, random norms) drive the act logits to about 30, which
    amplifies rounding: rounding GEMM operands, Q/K/V, P and the attention output to 16 bits in a
    CPU run of the oracle moves the logits by 1.07e-2 (fp16) and 0.145 (bf16).  The tolerances
    are about three and two times that (act logits: 0.142 and 1.13 in that run); the tight check
    at the usual weight scale is the test below."""
    spec = _modern_small(dtype)
    g = np.load(GOLDEN / "modernbert_small.npz")
    w = synthetic.weights(spec, seed=int(g["seed"]), random_norms=True, std=float(g["std"]))
    items = [(list(g[f"q{q}_ids"]), list(g[f"q{q}_markers"]), int(g[f"q{q}_kind"])) for q in range(int(g["n_q"]))]
    rt = Runtime(spec, 0, 4, weights=w)
    try:
        logits, acts, metrics = rt.predict(items)
        atol, acts_atol = (3e-2, 0.4) if dtype == "float16" else (0.3, 2.5)
        golden = [g[f"q{q}_logits"] for q in range(len(items))]
        compare(logits, acts, golden, np.stack([g[f"q{q}_acts"] for q in range(len(items))]), atol, acts_atol,
                label=f"modernbert small {dtype} vs transformers golden")
        want, want_acts = _modern_oracle(spec, w, items)
        compare(logits, acts, want, want_acts, atol, acts_atol, label=f"modernbert small {dtype} vs oracle")
        assert metrics["graph_capture"] and metrics["graph_replay"]
        eager = rt.predict(items, capture=False)
        np.testing.assert_array_equal(eager[0], logits)
        np.testing.assert_array_equal(eager[1], acts)
        # the GeGLU matrix is resident with interleaved rows; read-back returns checkpoint order
        name = "encoder.layers.1.mlp.Wi.weight"
        back = rt.weights[name].get()
        ref = w[name].astype(np.float16).astype(np.float32) if dtype == "float16" else synthetic.bf16_round(w[name])
        np.testing.assert_array_equal(back, ref)
    finally:
        rt.close()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_modernbert_small_at_checkpoint_scale_matches_oracle(gpu, dtype):
    """The same 4-layer, two-head-layer model at N(0, 0.02) weights with random norms: logits
    within 1e-3 (fp16) and 2e-3 (bf16) of the oracle, sequences long enough for the window to mask."""
    spec = _modern_small(dtype)
    w = synthetic.weights(spec, seed=21, random_norms=True)
    rng = np.random.default_rng(22)
    items = [(list(rng.integers(5, 1000, n)), sorted(rng.choice(np.arange(1, n), c, replace=False).tolist()), kind)
             for n, c, kind in ((400, 5, 1), (129, 3, 0), (33, 2, 2))]
    want, want_acts = _modern_oracle(spec, w, items)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        logits, acts, _ = rt.predict(items)
        compare(logits, acts, want, want_acts, atol=LOGIT_ATOL if dtype == "float16" else 2e-3,
                label=f"modernbert small {dtype} at checkpoint scale")
    finally:
        rt.close()


def test_modernbert_base_shaped_encoder_matches_oracle(gpu):
    """ModernBERT-base widths (d 768, 12 heads, GeGLU 1152) with 6 layers (global 0 and 3), two
    questions of 300 and 190 tokens packed back to back, one head layer: logits within 1e-3."""
    spec = synthetic.modernbert_adapter(layers=6, width=768, heads=12, intermediate=1152, vocab=50368,
                                        positions=8192, max_len=512, head_layers=1)
    w = synthetic.weights(spec, seed=9)
    rng = np.random.default_rng(10)
    items = [(list(rng.integers(5, 50368, 300)), sorted(rng.choice(np.arange(1, 300), 6, replace=False).tolist()), 0),
             (list(rng.integers(5, 50368, 190)), sorted(rng.choice(np.arange(1, 190), 4, replace=False).tolist()), 2)]
    want, want_acts = _modern_oracle(spec, w, items)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        logits, acts, _ = rt.predict(items)
        compare(logits, acts, want, want_acts, label="modernbert 6L/768")
    finally:
        rt.close()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_batched_modernbert_matches_oracle(gpu, dtype):
    """The ModernBERT variant in a batched slot (more than 4,096 packed rows): pre-LN layers whose
    out/down projections reach the residual as 16-bit rows, the GeGLU and RoPE epilogues on the
    large tiles, the LDS-shared attention with the +-64 window on local layers, and two head layers
    over every row; nine questions of 300-1,000 tokens, each its own sequence.  Tolerances as for
    the batch-1 workloads (fp16 1e-3, bf16 2e-3)."""
    spec = synthetic.modernbert_adapter(layers=4, width=256, heads=4, intermediate=512, vocab=3000, positions=1024,
                                        max_len=1024, head_layers=2, mfma_dtype=dtype)
    w = synthetic.weights(spec, seed=13, random_norms=True)
    rng = np.random.default_rng(14)
    items = [(list(rng.integers(5, 3000, int(n))), sorted(rng.choice(np.arange(1, int(n)), 5, replace=False).tolist()),
              i % 3) for i, n in enumerate(rng.integers(300, 1001, 9))]
    want, want_acts = _modern_oracle(spec, w, items)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        logits, acts, metrics = rt.predict(items)
        assert metrics["shape"][0] >= 4096, metrics["shape"]
        compare(logits, acts, want, want_acts, atol=LOGIT_ATOL if dtype == "float16" else 2e-3,
                label=f"batched modernbert {dtype} rows {metrics['shape'][0]}")
    finally:
        rt.close()


def test_large_batched_modernbert_matches_oracle(gpu):
    """A batched slot past 12,288 packed rows, where the out and down projections may run on
    hipBLASLt's kernels (chosen by timing when the slot is created; ModernBERT's have no bias):
    eighteen questions of 500-1,000 tokens, fp16 logits within 1e-3 of the oracle, and the graph
    replay equal to the eager forward bit for bit."""
    spec = synthetic.modernbert_adapter(layers=3, width=256, heads=4, intermediate=512, vocab=3000, positions=1024,
                                        max_len=1024, head_layers=1)
    w = synthetic.weights(spec, seed=17, random_norms=True)
    rng = np.random.default_rng(18)
    items = [(list(rng.integers(5, 3000, int(n))), sorted(rng.choice(np.arange(1, int(n)), 4, replace=False).tolist()),
              i % 3) for i, n in enumerate(rng.integers(500, 1001, 18))]
    want, want_acts = _modern_oracle(spec, w, items)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        logits, acts, metrics = rt.predict(items)
        assert metrics["shape"][0] >= 12288 and metrics["graph_replay"], metrics["shape"]
        eager = rt.predict(items, capture=False)
        np.testing.assert_array_equal(eager[0], logits)
        np.testing.assert_array_equal(eager[1], acts)
        compare(logits, acts, want, want_acts, label=f"batched modernbert rows {metrics['shape'][0]}")
    finally:
        rt.close()


def test_modernbert_base_shaped_encoder_at_1000_tokens_matches_oracle(gpu):
    """The same widths at the longest request a Laya checkpoint takes (max_len 1024,
    laya.py:101-107): a 1,000-token question and a 20-token one in one pack, so the batch-1 plan
    runs the paired split-key attention, with the +-64 window on the local layers (1, 2, 4, 5) and
    across the whole sequence on the global ones; logits within 1e-3."""
    spec = synthetic.modernbert_adapter(layers=6, width=768, heads=12, intermediate=1152, vocab=50368,
                                        positions=8192, max_len=1024, head_layers=1)
    w = synthetic.weights(spec, seed=11)
    rng = np.random.default_rng(12)
    items = [(list(rng.integers(5, 50368, 1000)), sorted(rng.choice(np.arange(1, 1000), 7, replace=False).tolist()), 1),
             (list(rng.integers(5, 50368, 20)), sorted(rng.choice(np.arange(1, 20), 3, replace=False).tolist()), 0)]
    want, want_acts = _modern_oracle(spec, w, items)
    rt = Runtime(spec, 0, 2, weights=w)
    try:
        logits, acts, metrics = rt.predict(items)
        assert metrics["shape"][0] >= 1024
        compare(logits, acts, want, want_acts, label="modernbert 6L/768 at 1,000 tokens")
    finally:
        rt.close()


def test_modernbert_rejects_mixed_types_on_a_shared_sequence(gpu):
    spec = synthetic.modernbert_adapter(layers=1, width=64, heads=1, intermediate=128, vocab=100, positions=128,
                                        max_len=64, head_layers=1)
    rt = Runtime(spec, 0, 1, weights=synthetic.weights(spec, seed=1))
    try:
        with pytest.raises(ValueError, match="share its type"):
            rt.predict_sequences([[1, 2, 3, 4]], [(0, [1], 0), (0, [2], 1)])
    finally:
        rt.close()


def test_stage_launch_counts_follow_the_variant(gpu):
    """Per-forward launch counts: encoder stages once per layer, head-layer stages once per head
    layer (the row gather only before the last), variant-only stages zero elsewhere."""
    bert = synthetic.adapter(None, layers=3, width=64, heads=1, intermediate=256, vocab=100, positions=64,
                             max_len=64)
    rt = Runtime(bert, 0, 1, weights=synthetic.weights(bert, seed=1))
    try:
        counts = {name: rt.stage_launches(name) for name in rt.stages()}
        assert counts["embed_norm"] == (1, 0) and counts["qkv"] == (3, 0)
        # the last layer's residual + LayerNorm runs inside the head gather, on the gathered rows only
        assert counts["ffn_norm"] == (2, 0)
        assert counts["head_gather"] == (1, 0) and counts["head_tail"] == (1, 0) and "act_out" not in counts
        assert counts["type_norm"] == (0, -1) and counts["head_qkv"] == (0, -1)
    finally:
        rt.close()
    modern = synthetic.modernbert_adapter(layers=2, width=64, heads=1, intermediate=128, vocab=100, positions=128,
                                          max_len=64, head_layers=3)
    rt = Runtime(modern, 0, 1, weights=synthetic.weights(modern, seed=1))
    try:
        counts = {name: rt.stage_launches(name) for name in rt.stages()}
        assert counts["qkv"] == (2, 0) and counts["type_norm"] == (1, 0) and counts["head_qkv"] == (3, 0)
        assert counts["head_gather_rows"] == (1, 2) and counts["head_gather"] == (0, -1)
        items = [(list(range(5, 45)), [3, 7], 1)]
        for name, (n, layer) in counts.items():
            if n:
                assert rt.time_stage([items[0][0]], [(0, items[0][1], 1)], name, layer, reps=2) > 0
    finally:
        rt.close()
