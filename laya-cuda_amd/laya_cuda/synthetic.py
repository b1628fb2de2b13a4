"""Seeded synthetic checkpoints and requests for the benchmark workloads.

No checkpoint or dataset can be downloaded, so every workload is generated:

* weights: NumPy PCG64 from ``seed`` (default 0), drawn in sorted-name order, N(0, 0.02) for
  matrices, embeddings and biases; LayerNorm gamma = 1, beta = 0 (or N(1,.1)/N(0,.1) with
  ``random_norms`` for kernel tests); ``bf16=True`` rounds every tensor to bfloat16 values;
* requests: NumPy PCG64 from ``seed`` (default 1).

Workloads (BERT-style post-LN encoder, d=64*heads, learned positions):
  ``l83``      12L/768, vocab 50,368, 512 positions, 1 sequence of 83 tokens, 1 question x 4 options
  ``l512``     same encoder, 512 tokens, 2 questions (4 and 6 options)
  ``l1024``    12L/768, vocab 250,002, 1024 positions, 1024 Zipf(1.1) tokens, 3 questions x 5 options
  ``ragged32`` 12L/768, 32 requests of U{40..900} tokens, 1-5 questions of 4-77 options each
  ``b64x1024`` 24L/1024, 16 heads, FFN 4096, bf16 weights, 64 x 1024 tokens, one 8-option question each
"""
import numpy as np

from .laya import Laya

WORKLOADS = {
    "l83": dict(layers=12, width=768, heads=12, intermediate=3072, vocab=50368, positions=512, max_len=512),
    "l512": dict(layers=12, width=768, heads=12, intermediate=3072, vocab=50368, positions=512, max_len=512),
    "l1024": dict(layers=12, width=768, heads=12, intermediate=3072, vocab=250002, positions=1024, max_len=1024),
    "ragged32": dict(layers=12, width=768, heads=12, intermediate=3072, vocab=50368, positions=1024, max_len=1024),
    "b64x1024": dict(layers=24, width=1024, heads=16, intermediate=4096, vocab=50368, positions=1024, max_len=1024,
                     bf16=True),
}


def encoder_config(layers, width, heads, intermediate, vocab, positions):
    return {"model_type": "bert", "hidden_size": width, "num_attention_heads": heads,
            "num_hidden_layers": layers, "intermediate_size": intermediate, "vocab_size": vocab,
            "max_position_embeddings": positions, "type_vocab_size": 2, "layer_norm_eps": 1e-12,
            "hidden_act": "gelu", "pad_token_id": 0}


def task_config(max_len, mfma_dtype="float16"):
    return {"max_len": max_len, "head_max_len": max_len, "head_layers": 0, "act_costs": {"defer": 0.05},
            "temperature": [1, 1, 1], "mfma_dtype": mfma_dtype}


def modernbert_config(layers, width, heads, intermediate, vocab, positions, global_every=3, local_attention=128,
                      global_theta=160000.0, local_theta=10000.0, eps=1e-5):
    """encoder/config.json of a ModernBERT/mmBERT encoder (the reference executor's variant)."""
    return {"model_type": "modernbert", "hidden_size": width, "num_attention_heads": heads,
            "num_hidden_layers": layers, "intermediate_size": intermediate, "vocab_size": vocab,
            "max_position_embeddings": positions, "global_attn_every_n_layers": global_every,
            "local_attention": local_attention, "global_rope_theta": global_theta, "local_rope_theta": local_theta,
            "norm_eps": eps, "norm_bias": False, "attention_bias": False, "mlp_bias": False,
            "hidden_activation": "gelu", "pad_token_id": 0}


def modernbert_adapter(*, layers, width, heads, intermediate, vocab, positions, max_len, head_layers=1,
                       mfma_dtype="float16", **config):
    """Checkpoint-less adapter of the ModernBERT variant with `head_layers` head transformer layers."""
    task = task_config(max_len, mfma_dtype)
    task["head_layers"] = head_layers
    return Laya.from_configs(modernbert_config(layers, width, heads, intermediate, vocab, positions, **config),
                             task, pad=0)


def adapter(name=None, *, mfma_dtype="float16", **overrides):
    """Checkpoint-less adapter for a named workload (or explicit sizes)."""
    spec = dict(WORKLOADS[name]) if name else {}
    spec.update(overrides)
    spec.pop("bf16", None)
    config = encoder_config(spec["layers"], spec["width"], spec["heads"], spec["intermediate"], spec["vocab"],
                            spec["positions"])
    return Laya.from_configs(config, task_config(spec["max_len"], mfma_dtype), pad=0)


def bf16_round(array):
    """Round float32 values to the nearest bfloat16 (ties to even), kept as float32."""
    bits = np.ascontiguousarray(array, np.float32).view(np.uint32)
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return rounded.view(np.float32)


def weights(spec, seed=0, *, random_norms=False, bf16=False, std=0.02):
    """{name: float32 array} for ``spec.weight_shapes()``, drawn in sorted-name order."""
    rng = np.random.default_rng(seed)
    std = np.float32(std)
    out = {}
    for name, shape in sorted(spec.weight_shapes().items()):
        if name == "temperature":
            out[name] = np.ones(shape, np.float32)
            continue
        norm = ("norm" in name or name.startswith("scorer.0.")) and len(shape) == 1
        if norm and name.endswith(".weight"):
            value = (rng.normal(1, .1, shape).astype(np.float32) if random_norms else np.ones(shape, np.float32))
        elif norm:
            value = (rng.normal(0, .1, shape).astype(np.float32) if random_norms else np.zeros(shape, np.float32))
        else:
            value = rng.standard_normal(shape, dtype=np.float32) * std
        out[name] = bf16_round(value) if bf16 else value
    return out


def _markers(rng, length, count, replace=False):
    population = np.arange(1, length)
    if not replace and count > len(population):
        replace = True
    return sorted(int(x) for x in rng.choice(population, count, replace=replace))


def zipf_ids(rng, n, vocab, s=1.1, first=5):
    """ids = first + perm(r-1), r ~ Zipf(s) truncated to [1, vocab-first] by inverse CDF."""
    ranks = np.arange(1, vocab - first + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="left")
    perm = rng.permutation(vocab - first)
    return (first + perm[r]).astype(np.int32)


def request(name, seed=1, **overrides):
    """(sequences, questions) of a workload; questions are (sequence index, markers, kind)."""
    spec = dict(WORKLOADS[name])
    spec.update(overrides)
    rng = np.random.default_rng(seed)
    vocab = spec["vocab"]
    if name == "l83":
        ids = rng.integers(5, vocab, 83, dtype=np.int32)
        return [ids], [(0, _markers(rng, 83, 4), 0)]
    if name == "l512":
        ids = rng.integers(5, vocab, 512, dtype=np.int32)
        return [ids], [(0, _markers(rng, 512, 4), 0), (0, _markers(rng, 512, 6), 0)]
    if name == "l1024":
        ids = zipf_ids(rng, 1024, vocab)
        return [ids], [(0, _markers(rng, 1024, 5), 0) for _ in range(3)]
    if name == "ragged32":
        lengths = rng.integers(40, 901, 32)
        sequences, questions = [], []
        for s, n in enumerate(lengths):
            sequences.append(rng.integers(5, vocab, int(n), dtype=np.int32))
            for _ in range(int(rng.integers(1, 6))):
                count = int(rng.integers(4, 78))
                questions.append((s, _markers(rng, int(n), count, replace=True), 0))
        return sequences, questions
    if name == "b64x1024":
        batch = spec.get("batch", 64)
        sequences = [rng.integers(5, vocab, 1024, dtype=np.int32) for _ in range(batch)]
        return sequences, [(s, _markers(rng, 1024, 8), 0) for s in range(batch)]
    raise KeyError(name)


def valid_flops(spec, lengths):
    """Algorithmic encoder FLOPs over valid tokens: per sequence of length L and layer,
    8 L d^2 + 4 L d f + 4 L^2 d (QKV 6Ld^2, out 2Ld^2, FFN 4Ldf, QK^T + PV 4L^2 d)."""
    d, f = spec.width, spec.intermediate
    return sum(spec.layers * (8 * L * d * d + 4 * L * d * f + 4 * L * L * d) for L in lengths)


# A small fixed corpus for the checkpoint tokenizer: support-ticket vocabulary plus the question
# scaffolding ("<type> question: ...", the noul defaults, score levels) that prepare() encodes.
TOKENIZER_CORPUS = [
    "refund the payment for the order", "choose a team for billing questions", "choose a topic",
    "the customer asks about a late delivery and wants a refund", "yes, the statement holds",
    "no, the statement does not hold", "level 0: not urgent", "level 1: urgent", "level 2: critical",
    "billing team handles invoices and payment errors", "shipping team handles delivery and tracking",
    "software questions go to the engineering queue", "other questions go to the general support queue",
    "noul question: is the customer angry?", "choice question: route the ticket",
    "score question: how urgent is the ticket?", "payment software ticket order customer delivery",
]
TOKENIZER_SPECIALS = ["[PAD]", "[UNK]", "[CLS]", "[SEP]", "[MASK]"]


def tokenizer(vocab_size=400):
    """Byte-pair tokenizer trained offline on TOKENIZER_CORPUS (whitespace pre-tokenizer; ids 0-4 are
    [PAD] [UNK] [CLS] [SEP] [MASK])."""
    from tokenizers import Tokenizer, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE(unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    tok.train_from_iterator(TOKENIZER_CORPUS * 10, trainers.BpeTrainer(vocab_size=vocab_size,
                                                                       special_tokens=TOKENIZER_SPECIALS))
    return tok


def checkpoint(root, config, task, *, seed=3, random_norms=True, bf16=False):
    """Write a complete checkpoint directory (model.safetensors, rl_agent_config.json,
    encoder/config.json, tokenizer/) for ``config``/``task`` with seeded weights; returns
    (path, adapter spec, weights).  ``config["vocab_size"]`` must cover the tokenizer's ids."""
    import json
    from pathlib import Path

    from safetensors.numpy import save_file
    root = Path(root)
    (root / "tokenizer").mkdir(parents=True, exist_ok=True)
    (root / "encoder").mkdir(exist_ok=True)
    tok = tokenizer()
    if tok.get_vocab_size() > config["vocab_size"]:
        raise ValueError("The encoder vocabulary must cover the tokenizer")
    tok.save(str(root / "tokenizer" / "tokenizer.json"))
    (root / "tokenizer" / "special_tokens_map.json").write_text(json.dumps(
        {"cls_token": "[CLS]", "sep_token": "[SEP]", "mask_token": "[MASK]", "pad_token": "[PAD]"}))
    (root / "encoder" / "config.json").write_text(json.dumps(config))
    (root / "rl_agent_config.json").write_text(json.dumps(task))
    spec = Laya.from_configs(config, task)
    flat = weights(spec, seed=seed, random_norms=random_norms, bf16=bf16)
    save_file({k: np.ascontiguousarray(v) for k, v in flat.items()}, str(root / "model.safetensors"))
    return root, spec, flat
