"""CPU emulation of the HIP encoder path's 16-bit rounding points (test infrastructure).

The oracle (oracle/encoder.py) runs the BERT-style forward in float32 throughout.  The GPU path
computes the same forward with 16-bit MFMA operands and fp32 accumulation, so its logits differ
from the oracle's by what those roundings add up to over the layers.  This module replays the
forward with exactly those rounding points, in NumPy, so that the error a given operand type
*must* show (independent of kernel bugs) can be stated before a tolerance is chosen:

* the normalised GEMM input ``x`` is stored as 16-bit after every LayerNorm (and the embedding
  norm); the fp32 residual stays fp32;
* every weight matrix is an MFMA operand of the chosen type (weights that are already bf16
  values are exact in bf16, and in fp16 down to 2^-17);
* Q, K and V leave the QKV GEMM rounded (bias added in fp32 before the rounding);
* attention: scores in fp32, probabilities rounded to 16 bits as the PV product's operand, the
  row sum taken over those rounded probabilities, the normalised output rounded;
* the FFN-up output is rounded after the fp32 GELU;
* the out and down projections are rounded to 16-bit rows (bias first) before the residual add
  when ``branch16`` (batched slots, the reference's half ``branch``), else summed in fp32 (the
  split-K partials of batch-1 slots);
* the decision head runs in fp32 on the final fp32 residual rows.

``python tests/rounding_emulation.py`` prints the emulated error of both operand types on the
24-layer d=1024 batch's first sequences against the FP32 oracle.
"""
import sys
from pathlib import Path

import numpy as np

if __name__ == "__main__":
    ROOT = Path(__file__).resolve().parents[1]
    sys.path[:0] = [str(ROOT), str(ROOT / "laya-cuda_amd")]

import oracle.encoder as E  # noqa: E402

F32 = np.float32


def bf16(x):
    """Round float32 values to the nearest bfloat16 (ties to even), kept as float32."""
    bits = np.ascontiguousarray(x, F32).view(np.uint32)
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return rounded.view(F32)


def f16(x):
    """Round float32 values to the nearest fp16 (ties to even), kept as float32."""
    return np.asarray(x, F32).astype(np.float16).astype(F32)


ROUND = {"float16": f16, "bfloat16": bf16, "none": lambda x: np.asarray(x, F32)}


def attention(q, k, v, r):
    """softmax(q k^T / 8) v per head with the PV operand and the output rounded by ``r``."""
    L, h, _ = q.shape
    qh, kh, vh = (np.ascontiguousarray(a.transpose(1, 0, 2)) for a in (q, k, v))
    s = np.matmul(qh, kh.transpose(0, 2, 1), dtype=F32) * F32(0.125)
    p = r(np.exp(s - s.max(-1, keepdims=True)))
    o = np.matmul(p, vh, dtype=F32) / p.sum(-1, keepdims=True, dtype=F32)
    return r(o.transpose(1, 0, 2).reshape(L, h * 64))


def encoder_sequence(ids, w, cfg, dtype, branch16=True):
    """The post-LN encoder of oracle.encoder.encoder_sequence with the GPU path's rounding points."""
    r = ROUND[dtype]
    d, heads, eps = cfg["width"], cfg["heads"], cfg["eps"]
    res = E.embed(ids, w, cfg)
    x = r(res)
    L = len(ids)
    for layer in w["layers"]:
        qkv = r(E._mm(x, r(layer["Wqkv"])) + layer["bqkv"])
        a = attention(qkv[:, :d].reshape(L, heads, 64), qkv[:, d:2 * d].reshape(L, heads, 64),
                      qkv[:, 2 * d:].reshape(L, heads, 64), r)
        branch = E._mm(a, r(layer["Wo"])) + layer["bo"]
        res = E.layer_norm(res + (r(branch) if branch16 else branch), layer["attn_norm_w"], layer["attn_norm_b"], eps)
        x = r(res)
        ff = r(E.gelu(E._mm(x, r(layer["Wi"])) + layer["bi"]))
        branch = E._mm(ff, r(layer["Wo2"])) + layer["bo2"]
        res = E.layer_norm(res + (r(branch) if branch16 else branch), layer["mlp_norm_w"], layer["mlp_norm_b"], eps)
        x = r(res)
    return res


def logit_error(spec, weights, sequences, questions, dtype, branch16=True):
    """Max |emulated logit - FP32 oracle logit| over the questions, and the questions whose argmax
    differs."""
    cfg = {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers}
    w = E.structured(weights, cfg)
    worst, flips = 0.0, []
    hidden = {}
    for q, (seq, markers, kind) in enumerate(questions):
        if seq not in hidden:
            hidden[seq] = (E.encoder_sequence(sequences[seq], w, cfg),
                           encoder_sequence(sequences[seq], w, cfg, dtype, branch16))
        exact, emulated = hidden[seq]
        want = E.head(exact, markers, kind, w)[0]
        got = E.head(emulated, markers, kind, w)[0]
        worst = max(worst, float(np.abs(got - want).max()))
        if int(np.argmax(got)) != int(np.argmax(want)):
            flips.append(q)
    return worst, flips


def main():
    from laya_cuda import synthetic
    count = int(sys.argv[1]) if len(sys.argv) > 1 else 3
    for name, picks in (("b64x1024", [0, 37, 63][:count]), ("l512", None)):
        spec = synthetic.adapter(name)
        w = synthetic.weights(spec, seed=0, bf16=synthetic.WORKLOADS[name].get("bf16", False))
        sequences, questions = synthetic.request(name, seed=1)
        if picks is not None:
            questions = [questions[p] for p in picks]
        for dtype in ("float16", "bfloat16"):
            for branch16 in ((True,) if name == "b64x1024" else (False,)):
                worst, flips = logit_error(spec, w, sequences, questions, dtype, branch16)
                print(f"{name} {dtype} branch16={branch16}: max |logit error| {worst:.3e}, flips {flips}",
                      flush=True)


if __name__ == "__main__":
    main()
