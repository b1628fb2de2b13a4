"""NumPy FP32 restatement of the reference's ModernBERT executor.  TEST INFRASTRUCTURE (the oracle).

Not product code: imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.

This is the variant laya-cuda runs for real Laya checkpoints (laya_cuda/laya.py:54-99,
laya_cuda/runtime.py:90-109): pre-LN blocks, LayerNorm without bias, RoPE on Q and K (rotate-half,
theta 160000 for global layers and 10000 for local ones), a +-window mask on local layers (every
layer whose index is not a multiple of ``global_every``), GeGLU FFN, no biases in the encoder, a
final norm; then the decision head's torch-style transformer layers (laya.py:214-235: norm1 ->
in_proj -> attention -> out_proj -> residual, norm2 -> linear1 -> ReLU -> linear2 -> residual)
before the same scorer, features and act head as the BERT-style variant.  Sequences are unpacked,
one per question, positions 0..L-1.  The block order is pinned by transformers' ModernBertModel
and torch's TransformerEncoderLayer(norm_first=True) fixtures in tests/golden/.
"""
import numpy as np

from . import encoder as E

F32 = np.float32


def rope_tables(theta, positions):
    """cos/sin [positions][32] exactly as the reference builds them (runtime.py:159-165):
    freq = 1/theta^(2i/64) and angle = pos * freq, all in float32."""
    freq = F32(1) / (F32(theta) ** (np.arange(0, 64, 2, dtype=F32) / F32(64)))
    angle = np.arange(positions, dtype=np.int32)[:, None].astype(F32) * freq
    return np.cos(angle).astype(F32), np.sin(angle).astype(F32)


def rope(x, cos, sin):
    """Rotate-half RoPE over [L, h, 64] (layout kernel, kernels.cu:73-77): for d < 32,
    x'[d] = x[d] cos - x[d+32] sin and x'[d+32] = x[d+32] cos + x[d] sin."""
    x = np.asarray(x, F32)
    c, s = cos[:, None, :], sin[:, None, :]
    lo, hi = x[..., :32], x[..., 32:]
    return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=-1).astype(F32)


def layer_norm(x, gamma, eps, beta=None):
    return E.layer_norm(x, gamma, beta, eps)


def encoder_sequence(ids, w, cfg):
    """Final hidden state [L, d] of one sequence (runtime.py:90-109)."""
    d, heads, eps = cfg["width"], cfg["heads"], cfg["eps"]
    L = len(ids)
    h = layer_norm(w["tok"][np.asarray(ids, np.int64)], w["emb_norm"], eps)
    for i, ly in enumerate(w["layers"]):
        x = h if i == 0 else layer_norm(h, ly["attn_norm"], eps)
        qkv = E._mm(x, ly["Wqkv"])
        q = qkv[:, :d].reshape(L, heads, 64)
        k = qkv[:, d:2 * d].reshape(L, heads, 64)
        v = qkv[:, 2 * d:].reshape(L, heads, 64)
        local = i % cfg["global_every"] != 0
        cos, sin = rope_tables(cfg["theta"][int(local)], L)
        a = E.attention(rope(q, cos, sin), rope(k, cos, sin), v, cfg["window"] if local else -1)
        h = h + E._mm(a, ly["Wo"])
        x = layer_norm(h, ly["mlp_norm"], eps)
        u = E._mm(x, ly["Wi"])
        f = u.shape[1] // 2
        h = h + E._mm((E.gelu(u[:, :f]) * u[:, f:]).astype(F32), ly["Wo2"])
    return layer_norm(h, w["final_norm"], eps)


def head_layers(h, kind, w, cfg):
    """Question-type row plus the head's transformer layers over one question's rows
    (laya.py:218-235); returns the final rows [L, d]."""
    hd = w["head"]
    heads, L = cfg["heads"], h.shape[0]
    d = h.shape[1]
    h = (h + hd["type_emb"][kind]).astype(F32)
    for ly in w["head_layers"]:
        x = layer_norm(h, ly["norm1_w"], 1e-5, ly["norm1_b"])
        qkv = E._mm(x, ly["in_w"]) + ly["in_b"]
        q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(L, heads, 64) for j in range(3))
        h = h + (E._mm(E.attention(q, k, v), ly["out_w"]) + ly["out_b"])
        x = layer_norm(h, ly["norm2_w"], 1e-5, ly["norm2_b"])
        ff = np.maximum(E._mm(x, ly["l1_w"]) + ly["l1_b"], F32(0))
        h = (h + (E._mm(ff, ly["l2_w"]) + ly["l2_b"])).astype(F32)
    return h


def head(rows_out, markers, w):
    """Scorer, features and act head on rows that already carry the question type
    (laya.py:236-245); same arithmetic as the BERT-style head with a zero type row."""
    zero = dict(w["head"], type_emb=np.zeros_like(w["head"]["type_emb"]))
    return E.head(rows_out, markers, 0, {"head": zero})


def forward(items, w, cfg):
    """Reference-style items [(ids, markers, kind)], one sequence per question (runtime.py:52-68).
    Returns (logits list [count], acts [n, n_act], hidden list)."""
    logits, acts, hidden = [], [], []
    for ids, markers, kind in items:
        hs = encoder_sequence(ids, w, cfg)
        out = head_layers(hs, kind, w, cfg)
        lg, ac, _ = head(out, markers, w)
        logits.append(lg)
        acts.append(ac)
        hidden.append(hs)
    return logits, np.stack(acts).astype(F32), hidden


def structured(weights, cfg):
    """Group a flat ModernBERT-variant checkpoint (reference names, laya.py:167-190)."""
    g = lambda n: np.asarray(weights[n], F32)
    out = {"tok": g("encoder.embeddings.tok_embeddings.weight"), "emb_norm": g("encoder.embeddings.norm.weight"),
           "final_norm": g("encoder.final_norm.weight"), "layers": [], "head_layers": []}
    for i in range(cfg["layers"]):
        p = f"encoder.layers.{i}."
        out["layers"].append({
            "attn_norm": g(p + "attn_norm.weight") if i else None, "Wqkv": g(p + "attn.Wqkv.weight"),
            "Wo": g(p + "attn.Wo.weight"), "mlp_norm": g(p + "mlp_norm.weight"),
            "Wi": g(p + "mlp.Wi.weight"), "Wo2": g(p + "mlp.Wo.weight")})
    for i in range(cfg["head_layers"]):
        p = f"head.layers.{i}."
        out["head_layers"].append({
            "norm1_w": g(p + "norm1.weight"), "norm1_b": g(p + "norm1.bias"),
            "in_w": g(p + "self_attn.in_proj_weight"), "in_b": g(p + "self_attn.in_proj_bias"),
            "out_w": g(p + "self_attn.out_proj.weight"), "out_b": g(p + "self_attn.out_proj.bias"),
            "norm2_w": g(p + "norm2.weight"), "norm2_b": g(p + "norm2.bias"),
            "l1_w": g(p + "linear1.weight"), "l1_b": g(p + "linear1.bias"),
            "l2_w": g(p + "linear2.weight"), "l2_b": g(p + "linear2.bias")})
    out["head"] = {
        "type_emb": g("type_emb.weight"), "s0_w": g("scorer.0.weight"), "s0_b": g("scorer.0.bias"),
        "s1_w": g("scorer.1.weight"), "s1_b": g("scorer.1.bias"),
        "s3_w": g("scorer.3.weight"), "s3_b": g("scorer.3.bias"),
        "a0_w": g("act_head.0.weight"), "a0_b": g("act_head.0.bias"),
        "a2_w": g("act_head.2.weight"), "a2_b": g("act_head.2.bias")}
    return out


def config(spec):
    """Oracle configuration from a ModernBERT-variant adapter (laya_cuda.laya.EncoderSpec)."""
    return {"width": spec.width, "heads": spec.heads, "eps": spec.eps, "layers": spec.layers,
            "global_every": spec.global_every, "window": spec.window, "theta": list(spec.theta),
            "head_layers": spec.head_layers}
