"""Laya checkpoint and request contract: configuration, request preparation and decoding.

Behaviour follows laya_cuda/laya.py of the reference: question parsing (laya.py:21-45),
host softmax (48-51), preparation (104-135), decoding and answer structure (137-165) and the
weight table (167-190).  GPU work lives in liblaya_hip; this module never touches the device.

Two encoder variants are described:
  * ``modernbert`` - the reference's executor (pre-LN, RoPE, GeGLU, local/global attention,
    torch-style head layers); its weight table is the reference's;
  * ``bert``       - the BERT-style post-LN encoder with learned positions, dense GELU FFN and
    biases that the synthetic workloads use, with the same Laya decision head.
"""
import hashlib
import json
import math

import numpy as np

from .models import read_json

TYPES = ("choice", "score", "noul")

# Tokenizer stages that act character by character or only split (never join text across a split),
# and the pre-tokenizers among them that always split in front of a space that follows a letter or
# digit.  With such a configuration, and no added token that contains whitespace or strips the
# whitespace after it, a text cut at such spaces encodes piece by piece to the ids of the whole text:
# each piece after the first starts with that space exactly as it does inside the whole text.
_LOCAL_NORMALIZERS = {"NFC", "NFD", "NFKC", "NFKD", "Lowercase", "StripAccents", "BertNormalizer"}
_SPLITS_AT_SPACES = {"Whitespace", "WhitespaceSplit", "BertPreTokenizer"}
_LOCAL_PRE_TOKENIZERS = _SPLITS_AT_SPACES | {"Digits", "Punctuation", "UnicodeScripts", "ByteLevel", "Metaspace"}


def _splits_at_spaces(config):
    """True when the serialised tokenizer ``config`` (tokenizer.json) encodes a text cut in front of
    spaces that follow a letter or digit, piece by piece, to the whole text's ids."""
    def normalizer_ok(n):
        if n is None:
            return True
        if n.get("type") == "Sequence":
            return all(normalizer_ok(m) for m in n.get("normalizers", []))
        return n.get("type") in _LOCAL_NORMALIZERS

    def splits(p):
        t = p.get("type")
        return (t in _SPLITS_AT_SPACES or (t == "ByteLevel" and p.get("use_regex", True))
                or (t == "Metaspace" and p.get("split", True)))

    pre = config.get("pre_tokenizer")
    if pre is None or not normalizer_ok(config.get("normalizer")):
        return False
    parts = pre.get("pretokenizers", []) if pre.get("type") == "Sequence" else [pre]
    if not parts or not all(p.get("type") in _LOCAL_PRE_TOKENIZERS for p in parts) or not any(map(splits, parts)):
        return False
    if config.get("model", {}).get("type") not in ("BPE", "WordPiece", "WordLevel", "Unigram"):
        return False
    return not any(a.get("rstrip") or any(c.isspace() for c in a.get("content", ""))
                   for a in config.get("added_tokens", []))


def text(value):
    return value if isinstance(value, str) else json.dumps(value, ensure_ascii=False, default=str)


def question(value):
    """(kind, instruction, criteria, option strings) of one question definition."""
    kind, instruction, criteria = value["type"], value["instructions"], value.get("criteria")
    if kind not in TYPES:
        raise ValueError(f"Unsupported question type: {kind}")
    if kind == "choice":
        if isinstance(criteria, list):
            criteria = dict.fromkeys(criteria)
        if not isinstance(criteria, dict) or any(not isinstance(key, str) for key in criteria):
            raise ValueError("Choice criteria must be a mapping or list of string labels")
        options = [key if detail in (None, "") else f"{key}: {text(detail)}" for key, detail in criteria.items()]
    elif kind == "score":
        if not isinstance(criteria, list):
            raise ValueError("Score criteria must be a list")
        options = [f"level {level}: {text(detail)}" for level, detail in enumerate(criteria)]
    else:
        criteria = criteria or {}
        if not isinstance(criteria, dict):
            raise ValueError("Noul criteria must be a mapping")
        defaults = {"false": "no, the statement does not hold", "true": "yes, the statement holds"}
        options = []
        for key in ("false", "true"):
            given = criteria.get(key)
            options.append(f"{key}: {defaults[key] if given in (None, '') else text(given)}")
    if not options:
        raise ValueError("Each question must have at least one option")
    if not isinstance(instruction, str):
        instruction = json.dumps(instruction)
    return kind, instruction, criteria, options


def softmax(values):
    """Float32 softmax over the last axis, max-subtracted."""
    values = np.asarray(values, np.float32)
    shifted = np.exp(values - values.max(axis=-1, keepdims=True))
    return shifted / shifted.sum(axis=-1, keepdims=True)


class EncoderSpec:
    """Architecture fields the runtime needs, from ``encoder/config.json`` + ``rl_agent_config.json``."""

    def __init__(self, config, task):
        c = config
        self.variant = c.get("model_type")
        if self.variant not in ("modernbert", "bert") or c.get("hidden_activation", c.get("hidden_act", "gelu")) != "gelu":
            raise ValueError("Only ModernBERT/mmBERT or BERT-style encoders with exact GELU are supported")
        self.width, self.heads = c["hidden_size"], c["num_attention_heads"]
        if self.width % self.heads or self.width // self.heads != 64:
            raise ValueError("v1 requires 64-wide attention heads")
        self.layers, self.intermediate = c["num_hidden_layers"], c["intermediate_size"]
        self.vocab = c["vocab_size"]
        if self.variant == "modernbert":
            if any(c.get(k, False) for k in ("attention_bias", "mlp_bias", "norm_bias", "rope_scaling")):
                raise ValueError("Biased or scaled-RoPE encoder variants are unsupported")
            self.global_every = c.get("global_attn_every_n_layers", 3)
            self.window = c.get("local_attention", 128) // 2
            expected = ["full_attention" if i % self.global_every == 0 else "sliding_attention"
                        for i in range(self.layers)]
            if c.get("layer_types", expected) != expected:
                raise ValueError("Unsupported attention topology")
            self.theta = []
            for kind, default in (("full_attention", 160000), ("sliding_attention", 10000)):
                rope = c.get("rope_parameters", {}).get(kind, {})
                if rope.get("rope_type", "default") != "default":
                    raise ValueError("Only default RoPE is supported")
                field = "global_rope_theta" if kind == "full_attention" else "local_rope_theta"
                self.theta.append(float(rope.get("rope_theta", c.get(field, default)) or self.theta[0]))
            self.eps = float(c.get("norm_eps", 1e-5))
            self.max_positions, self.type_vocab = c["max_position_embeddings"], 1
        else:
            self.global_every, self.window, self.theta = 1, -1, []
            self.eps = float(c.get("layer_norm_eps", 1e-12))
            self.max_positions, self.type_vocab = c["max_position_embeddings"], c.get("type_vocab_size", 2)
        self.ff_width = max(2 * self.intermediate, 4 * self.width)
        self.max_len, self.head_max_len = task["max_len"], task["head_max_len"]
        self.head_layers = task["head_layers"]
        self.n_act = len(task.get("act_costs", {})) + 1
        self.act_hidden = 256
        least_head = 1 if self.variant == "modernbert" else 0
        if not 0 < self.max_len <= min(1024, self.max_positions) or self.head_layers < least_head:
            raise ValueError("Invalid context budget or decision head")
        self.mfma_dtype = task.get("mfma_dtype", "float16")
        if self.mfma_dtype not in ("bfloat16", "float16"):
            raise ValueError("mfma_dtype must be 'bfloat16' or 'float16'")

    def weight_shapes(self):
        """Checkpoint tensor names and shapes (reference table: laya.py:167-190)."""
        w, f = self.width, self.intermediate
        shapes = {"encoder.embeddings.tok_embeddings.weight": (self.vocab, w),
                  "type_emb.weight": (3, w), "temperature": (3,),
                  "scorer.0.weight": (w,), "scorer.0.bias": (w,), "scorer.1.weight": (w, w),
                  "scorer.1.bias": (w,), "scorer.3.weight": (1, w), "scorer.3.bias": (1,),
                  "act_head.0.weight": (self.act_hidden, w + 4), "act_head.0.bias": (self.act_hidden,),
                  "act_head.2.weight": (self.n_act, self.act_hidden), "act_head.2.bias": (self.n_act,)}
        if self.variant == "modernbert":
            shapes.update({"encoder.embeddings.norm.weight": (w,), "encoder.final_norm.weight": (w,)})
            for i in range(self.layers):
                p = f"encoder.layers.{i}."
                shapes.update({p + "attn.Wqkv.weight": (3 * w, w), p + "attn.Wo.weight": (w, w),
                               p + "mlp.Wi.weight": (2 * f, w), p + "mlp.Wo.weight": (w, f),
                               p + "mlp_norm.weight": (w,)})
                if i:
                    shapes[p + "attn_norm.weight"] = (w,)
            for i in range(self.head_layers):
                p = f"head.layers.{i}."
                shapes.update({p + "self_attn.in_proj_weight": (3 * w, w), p + "self_attn.in_proj_bias": (3 * w,),
                               p + "self_attn.out_proj.weight": (w, w), p + "self_attn.out_proj.bias": (w,),
                               p + "linear1.weight": (4 * w, w), p + "linear1.bias": (4 * w,),
                               p + "linear2.weight": (w, 4 * w), p + "linear2.bias": (w,),
                               p + "norm1.weight": (w,), p + "norm1.bias": (w,),
                               p + "norm2.weight": (w,), p + "norm2.bias": (w,)})
        else:
            shapes.update({"encoder.embeddings.position_embeddings.weight": (self.max_positions, w),
                           "encoder.embeddings.token_type_embeddings.weight": (self.type_vocab, w),
                           "encoder.embeddings.norm.weight": (w,), "encoder.embeddings.norm.bias": (w,)})
            for i in range(self.layers):
                p = f"encoder.layers.{i}."
                shapes.update({p + "attn.Wqkv.weight": (3 * w, w), p + "attn.Wqkv.bias": (3 * w,),
                               p + "attn.Wo.weight": (w, w), p + "attn.Wo.bias": (w,),
                               p + "post_attn_norm.weight": (w,), p + "post_attn_norm.bias": (w,),
                               p + "mlp.Wi.weight": (f, w), p + "mlp.Wi.bias": (f,),
                               p + "mlp.Wo.weight": (w, f), p + "mlp.Wo.bias": (w,),
                               p + "post_mlp_norm.weight": (w,), p + "post_mlp_norm.bias": (w,)})
        return shapes

    @property
    def precision(self):
        return self.mfma_dtype


class Laya(EncoderSpec):
    """Adapter for a Laya checkpoint directory (model.safetensors, configs, tokenizer)."""

    def __init__(self, path):
        self.path = path
        self.cfg = read_json(path / "rl_agent_config.json")
        self.config = read_json(path / "encoder/config.json")
        super().__init__(self.config, self.cfg)
        from tokenizers import Tokenizer
        self.tokenizer = Tokenizer.from_file(str(path / "tokenizer/tokenizer.json"))
        self.tokenizer.no_padding()
        self.tokenizer.no_truncation()
        self.prefix_cut = _splits_at_spaces(json.loads(self.tokenizer.to_str()))
        specials = {}
        for name in ("tokenizer_config.json", "special_tokens_map.json"):
            if (path / "tokenizer" / name).is_file():
                specials.update(read_json(path / "tokenizer" / name))
        for key in ("cls", "sep", "mask", "pad"):
            token = specials.get(key + "_token")
            token = token.get("content") if isinstance(token, dict) else token
            value = self.tokenizer.token_to_id(token) if isinstance(token, str) else None
            if value is None:
                raise ValueError(f"Missing tokenizer special token: {key}")
            setattr(self, key, value)
            if key == "mask":
                self.mask_text = token

    @classmethod
    def from_configs(cls, config, task, pad=0):
        """Adapter without files (synthetic checkpoints fed pre-tokenised ids): no ``prepare``."""
        self = object.__new__(cls)
        self.path, self.cfg, self.config, self.tokenizer, self.prefix_cut = None, task, config, None, False
        EncoderSpec.__init__(self, config, task)
        self.pad = pad
        return self

    def encode(self, value):
        return self.tokenizer.encode(value.replace(self.mask_text, " "), add_special_tokens=False).ids

    def state_ids(self, text, need=None):
        """The state text's ids as far as prepare can use them: the whole text's, or at least their
        first ``need`` (default max_len).  The reference encodes the whole state and keeps its first
        max_len - 3 or fewer ids (laya.py:110-130), so a long state costs the tokenizer time for
        every character.  Where the tokenizer splits in front of a space that follows a letter or
        digit (``prefix_cut``), the text is encoded in pieces cut at such spaces, the first about
        5 x ``need`` characters, each next one sized for the ids still missing, until ``need`` ids
        are there: the pieces' ids joined are the whole text's, and the work never exceeds
        encoding the whole text."""
        encode = self.tokenizer.encode
        if not self.prefix_cut:
            return encode(text, add_special_tokens=False).ids
        need = self.max_len if need is None else need
        ids, start, chars = [], 0, 5 * need + 64
        while start < len(text) and len(ids) < need:
            end = text.find(" ", start + chars)
            while end > 0 and not text[end - 1].isalnum():
                end = text.find(" ", end + 1)
            end = end if end > 0 else len(text)
            ids += encode(text[start:end], add_special_tokens=False).ids
            start = end
            chars = (need - len(ids)) * start // max(len(ids), 1) * 5 // 4 + 64
        return ids

    def prepare(self, state, questions):
        """Token ids, option marker positions and type per question (laya.py:104-135)."""
        if not isinstance(questions, dict) or not questions:
            raise ValueError("Provide a nonempty mapping of questions")
        if self.tokenizer is None:
            raise RuntimeError("This adapter has no tokenizer; pass token ids to Runtime.predict")
        parsed = [question(definition) for definition in questions.values()]
        texts = [state if isinstance(state, str) else json.dumps(state, ensure_ascii=False)]
        for kind, instruction, _, options in parsed:
            texts.append(f"{kind} question: {instruction}")
            texts.extend(" " + option for option in options)
        texts = [t.replace(self.mask_text, " ") for t in texts]
        if len(texts) >= 12:
            encoded = [e.ids for e in self.tokenizer.encode_batch(texts[1:], add_special_tokens=False)]
        else:
            encoded = [self.tokenizer.encode(t, add_special_tokens=False).ids for t in texts[1:]]
        cursor, layouts = iter(encoded), []
        for qid, (kind, _, _, options) in zip(questions, parsed):
            head = next(cursor)
            opts = [[self.mask] + next(cursor)[:48] for _ in options]
            budget = self.head_max_len - sum(len(o) for o in opts)
            if budget < 16:
                cap = max(4, (self.head_max_len - 16) // len(opts))
                opts = [o[:cap] for o in opts]
                budget = self.head_max_len - sum(len(o) for o in opts)
            ids = [self.cls] + head[:max(8, budget)] + [self.sep]
            markers = []
            for opt in opts:
                markers.append(len(ids))
                ids.extend(opt)
            ids.append(self.sep)
            layouts.append((qid, kind, ids, markers))
        # The state's ids after every question's layout: only as many as the roomiest one takes.
        rooms = [max(0, self.max_len - len(ids) - 1) for _, _, ids, _ in layouts]
        state_ids = self.state_ids(texts[0], max(rooms))
        items = []
        for (qid, kind, ids, markers), room in zip(layouts, rooms):
            ids = (ids + state_ids[:room] + [self.sep])[:self.max_len]
            if markers[-1] >= len(ids):
                raise ValueError(f"Question {qid!r} exceeds the option token budget")
            items.append((ids, markers, TYPES.index(kind)))
        return items

    def decode(self, logits, acts, questions, items):
        """Answer dicts from option logits [n, k] and act logits [n, n_act] (laya.py:137-165)."""
        if not np.isfinite(logits).all() or not np.isfinite(acts).all():
            raise RuntimeError("Non-finite model output; no decision returned")
        actions, answers = softmax(acts), {}
        calibration = self.cfg.get("temperature_by_options", {})
        for row, (qid, definition) in enumerate(questions.items()):
            kind, _, criteria, options = question(definition)
            count, qt = len(options), TYPES.index(kind)
            bucket = "2" if count <= 2 else "3-5" if count <= 5 else "6-10" if count <= 10 else "11+"
            temp = calibration.get(f"{kind}:{bucket}", self.cfg.get("temperature", [1] * 3)[qt])
            try:
                temp = float(temp)
            except (TypeError, ValueError):
                temp = 1.0
            temp = float(np.clip(temp, .5, 5)) if math.isfinite(temp) else 1.0
            prob = softmax(logits[row, :count].astype(np.float32) / np.float32(temp))
            if count > 1:
                entropy = (prob * np.log(np.maximum(prob, 1e-12))).sum()
                conf = float(np.clip(1 + entropy / math.log(count), 0, 1))
            else:
                conf = 1.0
            answer = {"type": kind, "confidence": round(conf, 4),
                      "action": {"act_probability": round(float(actions[row, 0]), 4)}}
            if kind == "noul":
                answer.update(noul=round(float(prob[1]), 4), confidence=round(float(max(prob[1], 1 - prob[1])), 4))
            else:
                keys = list(criteria) if kind == "choice" else [str(i) for i in range(count)]
                answer["probabilities"] = {key: round(float(p), 4) for key, p in zip(keys, prob)}
                if kind == "choice":
                    answer["choice"] = keys[int(prob.argmax())]
                else:
                    answer.update(score=round(float(np.arange(count) @ prob), 4), legend=dict(zip(keys, criteria)))
            answers[qid] = answer
        return {"model": "laya-rl-agent", "answers": answers,
                "usage": {"input_tokens": sum(len(item[0]) for item in items), "output_tokens": 0}}

    def fingerprint(self, items):
        return hashlib.sha256(json.dumps(items, separators=(",", ":")).encode()).hexdigest()

    def official(self, device):
        raise ValueError("backend='official' needs the official Laya SDK on CUDA, which this ROCm build does not ship")
