"""CPU FP32 oracle for the encoder forward path.  TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker (or, for ``cpu_baseline``, as the timed CPU path it
is reported beside).  The product path (``laya_cuda``) never imports it and has no CPU fallback.

``oracle.encoder`` restates, in NumPy float32, what the reference computes on its GPU path
(laya_cuda/kernels.cu, laya_cuda/runtime.py, laya_cuda/ops.py, laya_cuda/laya.py), for the
BERT-style post-LN encoder variant the workloads use.  It runs every sequence *unpacked*, so the
packed GPU layout (16-token spans, shape slots, tile lists) is checked against an independent
layout.

Parity pins (each one a check that a plausible mistake fails):

* encoder: transformers ``BertModel`` (an independent implementation of the same post-LN,
  learned-position, exact-GELU, eps 1e-12 encoder) on seeded weights, fixtures in
  ``tests/golden/`` written by ``tests/golden/make_golden.py``;
* layer_norm / gelu / attention: float64 textbook forms, and ``torch.nn.functional`` in the
  fixtures;
* head (gather, scorer, features, act head): torch ``nn.LayerNorm``/``nn.Linear``/``F.gelu``/
  ``softmax`` in the fixtures, plus the gather's bit-exact definition (row copy);
* decode: the reference's own known-answer tests (tests/test_contract.py:42-94).
"""
