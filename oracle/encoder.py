"""NumPy FP32 restatement of the encoder forward path.  TEST INFRASTRUCTURE (the oracle).

Not product code: imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.

Every function runs on *unpacked* sequences (one array per sequence, positions 0..L-1), so the
GPU's packed layout is checked against a layout it does not share.  Arithmetic is float32
throughout, in the order the reference's kernels use; only the GEMMs go through BLAS (sgemm).

Encoder variant: BERT-style post-LN (``h = LN(h + sublayer(h))``), learned absolute positions,
token type 0, dense FFN with exact GELU, biases everywhere.  The reference's kernels provide
each building block (citations per function); the block *order* is pinned by transformers'
BertModel fixtures in tests/golden/.
"""
import math

import numpy as np
from scipy.special import erf

F32 = np.float32


def _mm(x, w):
    """``x @ w.T`` in float32 (the reference's GEMM orientation, laya_cuda/ops.py:58-64)."""
    return np.matmul(x, w.T, dtype=F32)


def layer_norm(x, gamma, beta, eps):
    """Two-pass LayerNorm over the last axis (laya_cuda/kernels.cu:32-48).

    mean = sum(v)/w, var = sum((v-mean)^2)/w, out = (v-mean) * rsqrt(var+eps) * gamma + beta.
    """
    x = np.asarray(x, F32)
    w = x.shape[-1]
    mean = x.sum(-1, keepdims=True, dtype=F32) / F32(w)
    centred = x - mean
    var = (centred * centred).sum(-1, keepdims=True, dtype=F32) / F32(w)
    inv = F32(1) / np.sqrt(var + F32(eps))
    out = centred * inv * np.asarray(gamma, F32)
    if beta is not None:
        out = out + np.asarray(beta, F32)
    return out.astype(F32)


def gelu(x):
    """Exact-erf GELU, activate mode 0 (laya_cuda/kernels.cu:64): 0.5*v*(1+erf(v/sqrt(2)))."""
    x = np.asarray(x, F32)
    return (F32(0.5) * x * (F32(1) + erf(x * F32(0.7071067811865475)).astype(F32))).astype(F32)


def softmax(values, axis=-1):
    """Max-subtracted float32 softmax (laya_cuda/laya.py:48-51)."""
    values = np.asarray(values, F32)
    e = np.exp(values - values.max(axis=axis, keepdims=True))
    return (e / e.sum(axis=axis, keepdims=True)).astype(F32)


def embed(ids, w, cfg):
    """Token-row gather plus learned position and type-0 rows, then LayerNorm.

    Gather semantics follow ``embed`` (laya_cuda/kernels.cu:16-19): ``out[t] = table[ids[t]]``,
    a plain row copy.  The BERT-style variant adds ``position[t]`` and ``type[0]`` in that order
    before the embeddings norm (runtime.py:93-94 applies that norm to the gathered rows).
    """
    ids = np.asarray(ids, np.int64)
    e = w["encoder.embeddings"]
    v = e["tok"][ids] + e["pos"][np.arange(len(ids))]
    v = v + e["type"][0]
    return layer_norm(v, e["norm_w"], e["norm_b"], cfg["eps"])


def attention(q, k, v, window=-1):
    """Bidirectional softmax(Q K^T / 8) V for one sequence, per head (kernels.cu:90-154).

    q, k, v: [L, h, 64] float32.  ``window >= 0`` masks |query - key| > window, as the
    reference's local layers do; every key of the sequence is visible otherwise.  Returns [L, h*64].
    """
    L, h, _ = q.shape
    qh, kh, vh = (np.ascontiguousarray(a.transpose(1, 0, 2)) for a in (q, k, v))
    s = np.matmul(qh, kh.transpose(0, 2, 1), dtype=F32) * F32(0.125)
    if window >= 0:
        far = np.abs(np.arange(L)[:, None] - np.arange(L)[None, :]) > window
        s = np.where(far[None], F32(-np.inf), s)
    p = softmax(s)
    o = np.matmul(p, vh, dtype=F32)
    return o.transpose(1, 0, 2).reshape(L, h * 64).astype(F32)


def encoder_sequence(ids, w, cfg):
    """Post-LN encoder over one unpacked sequence: returns the final hidden state [L, d] fp32.

    Per layer: ``h = LN(h + Wo attn(h Wqkv^T + bqkv) + bo)``, then
    ``h = LN(h + W2 gelu(h W1^T + b1) + b2)``.  The residual add and LN come from
    ``layer_norm`` (kernels.cu:20-49); the biased GEMMs from ops.py:58-66 (bias added once to
    the float32 accumulation).
    """
    d, heads = cfg["width"], cfg["heads"]
    x = embed(ids, w, cfg)
    L = len(ids)
    for layer in w["layers"]:
        qkv = _mm(x, layer["Wqkv"]) + layer["bqkv"]
        q = qkv[:, :d].reshape(L, heads, 64)
        k = qkv[:, d:2 * d].reshape(L, heads, 64)
        v = qkv[:, 2 * d:].reshape(L, heads, 64)
        a = attention(q, k, v)
        branch = _mm(a, layer["Wo"]) + layer["bo"]
        x = layer_norm(x + branch, layer["attn_norm_w"], layer["attn_norm_b"], cfg["eps"])
        ff = gelu(_mm(x, layer["Wi"]) + layer["bi"])
        branch = _mm(ff, layer["Wo2"]) + layer["bo2"]
        x = layer_norm(x + branch, layer["mlp_norm_w"], layer["mlp_norm_b"], cfg["eps"])
    return x


def features(cls_row, logits, count):
    """Per-question softmax statistics of ``features`` (laya_cuda/kernels.cu:167-183).

    ``logits`` are the question's option logits (slots 1..count).  Returns [d+4] float32:
    the CLS row, p1, p1-p2, entropy/log(max(n,2)), max(n,2)/255.
    """
    z = np.asarray(logits[:count], F32)
    p = softmax(z)
    order = np.sort(p)[::-1]
    p1 = order[0]
    p2 = order[1] if count > 1 else F32(0)
    entropy = -(p * np.log(np.maximum(p, F32(1e-9)))).sum(dtype=F32)
    n = max(count, 2)
    tail = np.array([p1, p1 - p2, entropy / F32(math.log(n)), F32(n) / F32(255)], F32)
    return np.concatenate([np.asarray(cls_row, F32), tail])


def head(hidden, markers, kind, w):
    """Decision head with no head transformer layers (laya_cuda/laya.py:214-245, head_layers=0).

    ``hidden``: the question's sequence final hidden state [L, d].  Rows gathered are the CLS
    row (position 0) and one row per marker (gather, kernels.cu:159-162), each plus
    ``type_emb[kind]`` (type_add, kernels.cu:155-158).  Scorer: LN(eps 1e-5) -> Linear+b -> GELU
    -> Linear(1)+b (laya.py:238-241).  Act head over ``features`` (laya.py:242-245).
    Returns (logits[count], acts[n_act], feats[d+4]).
    """
    h = w["head"]
    rows = np.concatenate([[0], np.asarray(markers, np.int64)])
    selected = hidden[rows] + h["type_emb"][kind]
    # Duplicate markers are legal and must score identically: BLAS may round identical rows
    # differently by their place in a block, so score each distinct row once and expand.
    distinct, back = np.unique(rows, return_inverse=True)
    unique_sel = hidden[distinct] + h["type_emb"][kind]
    normed = layer_norm(unique_sel, h["s0_w"], h["s0_b"], 1e-5)
    scored = gelu(_mm(normed, h["s1_w"]) + h["s1_b"])
    logits = (_mm(scored, h["s3_w"]) + h["s3_b"])[:, 0][back.reshape(-1)]
    count = len(markers)
    feats = features(selected[0], logits[1:], count)
    hidden_act = gelu(_mm(feats[None], h["a0_w"]) + h["a0_b"])
    acts = (_mm(hidden_act, h["a2_w"]) + h["a2_b"])[0]
    return logits[1:].astype(F32), acts.astype(F32), feats


def forward(sequences, questions, w, cfg):
    """Full forward over unpacked sequences.

    sequences: list of token-id lists.  questions: list of (seq_index, markers, kind).
    Returns (logits list per question [count], acts [nq, n_act], hidden list per sequence).
    """
    hidden = [encoder_sequence(ids, w, cfg) for ids in sequences]
    logits, acts = [], []
    for seq, markers, kind in questions:
        lg, ac, _ = head(hidden[seq], markers, kind, w)
        logits.append(lg)
        acts.append(ac)
    return logits, np.stack(acts).astype(F32), hidden


def structured(weights, cfg):
    """Group a flat ``{name: array}`` checkpoint (laya_cuda naming) for the functions above."""
    g = lambda n: np.asarray(weights[n], F32)
    p = "encoder.embeddings."
    out = {"encoder.embeddings": {
        "tok": g(p + "tok_embeddings.weight"), "pos": g(p + "position_embeddings.weight"),
        "type": g(p + "token_type_embeddings.weight"),
        "norm_w": g(p + "norm.weight"), "norm_b": g(p + "norm.bias")}, "layers": []}
    for i in range(cfg["layers"]):
        p = f"encoder.layers.{i}."
        out["layers"].append({
            "Wqkv": g(p + "attn.Wqkv.weight"), "bqkv": g(p + "attn.Wqkv.bias"),
            "Wo": g(p + "attn.Wo.weight"), "bo": g(p + "attn.Wo.bias"),
            "attn_norm_w": g(p + "post_attn_norm.weight"), "attn_norm_b": g(p + "post_attn_norm.bias"),
            "Wi": g(p + "mlp.Wi.weight"), "bi": g(p + "mlp.Wi.bias"),
            "Wo2": g(p + "mlp.Wo.weight"), "bo2": g(p + "mlp.Wo.bias"),
            "mlp_norm_w": g(p + "post_mlp_norm.weight"), "mlp_norm_b": g(p + "post_mlp_norm.bias")})
    out["head"] = {
        "type_emb": g("type_emb.weight"), "s0_w": g("scorer.0.weight"), "s0_b": g("scorer.0.bias"),
        "s1_w": g("scorer.1.weight"), "s1_b": g("scorer.1.bias"),
        "s3_w": g("scorer.3.weight"), "s3_b": g("scorer.3.bias"),
        "a0_w": g("act_head.0.weight"), "a0_b": g("act_head.0.bias"),
        "a2_w": g("act_head.2.weight"), "a2_b": g("act_head.2.bias")}
    return out
