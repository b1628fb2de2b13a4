"""Full-size parity of the two largest workloads on the GPU, against the CPU oracle.

* l1024: 12L/768 encoder with a 250,002-row fp32 embedding table (768 MB resident), one sequence
  of 1,024 Zipf(1.1) token ids, three 5-option questions; fp16 operands, logits within 1e-3 and
  identical decisions; embedding rows gathered from the whole table (its last rows included)
  bit for bit.
* b64x1024: 24L/1024 encoder, 16 heads, FFN 4096, bf16-valued weights, 64 x 1,024 dense tokens,
  one 8-option question per sequence.  The whole batch runs on the GPU; sequences are
  independent, so three of them (first, middle, last in the packed block) are checked against
  the oracle run on those sequences alone.  Graph replay equals the eager pass bit for bit.
  fp16 operands (the benchmarked mode) are held to the 1e-3 bound; bf16 operands to 4e-3.
"""
import ctypes as ct

import numpy as np
import pytest

from laya_cuda import _lib, synthetic
from laya_cuda.runtime import Runtime
from test_runtime_gpu import compare, oracle_logits

pytestmark = pytest.mark.gpu

# The 24-layer d=1024 batch.  Its weights are bf16 values by definition; fp16 holds every one of them
# exactly down to 2^-17 (N(0, 0.02) draws below that are rounded by less than 2^-25), so fp16
# operands add no weight rounding either.  A CPU emulation of this path's rounding points
# (tests/rounding_emulation.py: 16-bit normalised GEMM inputs, Q/K/V, attention probabilities and
# output, FFN activations, and the 16-bit out/down projection rows added to the fp32 residual)
# gives a max logit error on sequences 0, 37 and 63 of 2.78e-4 with fp16 operands and 2.85e-3 with
# bf16: bf16 cannot meet the 1e-3 bound on this model, fp16 meets it with room.
B64_LOGIT_ATOL = {"float16": 1e-3, "bfloat16": 4e-3}
B64_PICKS = [0, 37, 63]
_b64_oracle = {}


def test_l1024_large_vocab_matches_oracle(gpu):
    import torch
    spec = synthetic.adapter("l1024", mfma_dtype="float16")
    w = synthetic.weights(spec, seed=0)
    sequences, questions = synthetic.request("l1024", seed=1)
    ids = sequences[0]
    assert len(ids) == 1024 and spec.vocab == 250002
    want, want_acts = oracle_logits(spec, w, sequences, questions)
    rt = Runtime(spec, 0, 1, weights=w)
    try:
        logits, acts, metrics = rt.predict_sequences(sequences, questions)
        assert metrics["shape"] == (1024, 4, 8) and metrics["graph_replay"]
        compare(logits, acts, want, want_acts, label="l1024 fp16")
        eager = rt.predict_sequences(sequences, questions, capture=False)
        np.testing.assert_array_equal(eager[0], logits)
        np.testing.assert_array_equal(eager[1], acts)
    finally:
        rt.close()
    # Embedding gather over the whole 250,002-row table: the request's Zipf ids plus the table's
    # last rows and a few duplicates, bit for bit (no position or type row, no LayerNorm).
    lib = _lib.load()
    table = torch.from_numpy(w["encoder.embeddings.tok_embeddings.weight"]).to(gpu)
    pick = np.concatenate([ids, np.arange(spec.vocab - 16, spec.vocab), [spec.vocab - 1, 5, 5]]).astype(np.int32)
    positions = np.zeros(len(pick), np.int32)
    d_ids, d_pos = (torch.from_numpy(a).to(gpu) for a in (pick, positions))
    out = torch.full((len(pick), spec.width), float("nan"), device=gpu)
    _lib.check(lib.laya_op_embed(ct.c_void_p(d_ids.data_ptr()), ct.c_void_p(d_pos.data_ptr()),
                                 ct.c_void_p(table.data_ptr()), None, None, None, None, 0.0,
                                 ct.c_void_p(out.data_ptr()), None, _lib.F16, len(pick), spec.width, spec.vocab, 1,
                                 ct.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    host = w["encoder.embeddings.tok_embeddings.weight"]
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), host[pick].view(np.uint32))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_b64x1024_batch_matches_oracle_on_sampled_sequences(gpu, dtype):
    spec = synthetic.adapter("b64x1024", mfma_dtype=dtype)
    w = synthetic.weights(spec, seed=0, bf16=True)
    sequences, questions = synthetic.request("b64x1024", seed=1)
    assert len(sequences) == 64 and all(len(s) == 1024 for s in sequences)
    rt = Runtime(spec, 0, 1, weights=w)
    try:
        logits, acts, metrics = rt.predict_sequences(sequences, questions)
        assert metrics["shape"] == (65536, 64, 8) and metrics["graph_replay"]
        assert np.isfinite(logits).all() and np.isfinite(acts).all()
        eager = rt.predict_sequences(sequences, questions, capture=False)
        np.testing.assert_array_equal(eager[0], logits)
        np.testing.assert_array_equal(eager[1], acts)
    finally:
        rt.close()
    if not _b64_oracle:  # the oracle does not depend on the operand type: computed once
        sub_seqs = [sequences[i] for i in B64_PICKS]
        sub_qs = [(j, questions[i][1], questions[i][2]) for j, i in enumerate(B64_PICKS)]
        _b64_oracle["want"] = oracle_logits(spec, w, sub_seqs, sub_qs)
    want, want_acts = _b64_oracle["want"]
    compare(logits[B64_PICKS], acts[B64_PICKS], want, want_acts, atol=B64_LOGIT_ATOL[dtype],
            label=f"b64x1024 {dtype} (sequences 0, 37, 63)")
