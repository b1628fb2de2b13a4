"""Host-side request/answer contract (no GPU): what `Laya.question`, `softmax` and `Laya.decode`
produce for fixed inputs, which inputs they refuse, and what importing the package costs.

The known answers (expected option texts, probabilities and messages) are the reference's
published behaviour (tests/test_contract.py:11-94 of laya-cuda), kept here as data tables; each
test derives its expectation independently where it can (float64 arithmetic, the temperature
rule written out) rather than repeating the decode code.
"""
import json
import math
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from laya_cuda.laya import TYPES, Laya, question, softmax

ROOT = Path(__file__).resolve().parents[1]

# ---- data: question definitions and the option texts / instruction text they must produce ----
OPTION_TEXTS = [
    ({"type": "choice", "instructions": {"ask": "team"}, "criteria": {"no": False, "zero": 0, "empty": None}},
     ["no: false", "zero: 0", "empty"]),
    ({"type": "noul", "instructions": "yes?"},
     ["false: no, the statement does not hold", "true: yes, the statement holds"]),
    ({"type": "score", "instructions": "x", "criteria": ["low", {"a": 1}]},
     ["level 0: low", 'level 1: {"a": 1}']),
]
INSTRUCTION_TEXTS = [({"type": "choice", "instructions": ["a"], "criteria": ["x"]}, '["a"]')]
REFUSED_QUESTIONS = [
    ({"type": "choice", "instructions": "x", "criteria": []}, None),
    ({"type": "rank", "instructions": "x"}, "Unsupported question type"),
    ({"type": "score", "instructions": "x", "criteria": {"a": 1}}, "Score criteria"),
]
HEAVY_MODULES = ["torch", "transformers", "cupy", "psutil", "pyarrow"]


def bare_adapter(task):
    """A Laya whose decode can run: only the task configuration is set."""
    adapter = object.__new__(Laya)
    adapter.cfg = task
    return adapter


def probabilities64(logits, temperature):
    """Reference arithmetic written independently: softmax in float64 of logits / temperature."""
    z = np.asarray(logits, np.float64) / temperature
    e = np.exp(z - z.max())
    return e / e.sum()


def test_importing_the_package_loads_no_heavy_module():
    probe = (f"import sys, json; sys.path.insert(0, {str(ROOT / 'laya-cuda_amd')!r}); import laya_cuda; "
             f"print(json.dumps([sorted(set({HEAVY_MODULES!r}) & set(sys.modules)), sorted(laya_cuda.__all__)]))")
    loaded, exported = json.loads(subprocess.run([sys.executable, "-c", probe], check=True, capture_output=True,
                                                 text=True).stdout)
    assert loaded == []
    assert exported == ["BatchEngine", "Engine"]


def test_native_sources_are_ascii():
    for path in (ROOT / "laya-cuda_amd" / "csrc").glob("*.[hc]*"):
        assert path.read_bytes().isascii(), path
    assert (ROOT / "include" / "laya_hip.h").read_bytes().isascii()


@pytest.mark.parametrize("definition,texts", OPTION_TEXTS, ids=["choice-dict", "noul-default", "score-list"])
def test_option_texts(definition, texts):
    kind, _, _, options = question(definition)
    assert kind == definition["type"] and options == texts


@pytest.mark.parametrize("definition,text", INSTRUCTION_TEXTS)
def test_instruction_text_of_non_string_instructions(definition, text):
    assert question(definition)[1] == text


@pytest.mark.parametrize("definition,message", REFUSED_QUESTIONS, ids=["no-criteria", "unknown-type", "score-dict"])
def test_refused_questions(definition, message):
    with pytest.raises(ValueError, match=message):
        question(definition)


@pytest.mark.parametrize("logits", [[1e4, 1e4], [-1e4, -1e4, -1e4], [88.0, 88.0, 88.0, 88.0]])
def test_softmax_of_equal_extreme_logits_is_uniform(logits):
    p = softmax(logits)
    assert p.dtype == np.float32 and np.isfinite(p).all()
    np.testing.assert_allclose(p, np.full(len(logits), 1 / len(logits)), rtol=1e-6)


def test_softmax_is_shift_invariant_and_normalised():
    rng = np.random.default_rng(4)
    z = rng.normal(0, 3, (5, 9)).astype(np.float32)
    np.testing.assert_allclose(softmax(z), softmax(z + 37), atol=1e-5)
    np.testing.assert_allclose(softmax(z).sum(-1), 1, atol=1e-6)
    np.testing.assert_allclose(softmax(z), [probabilities64(row, 1.0) for row in z], atol=1e-6)


def test_one_option_is_certain_and_neutral_act():
    adapter = bare_adapter({"temperature": [1, 1, 1]})
    single = {"q": {"type": "choice", "instructions": "choose", "criteria": ["only"]}}
    out = adapter.decode(np.array([[7.0]]), np.zeros((1, 2)), single, [([1, 2], [1], 0)])
    answer = out["answers"]["q"]
    assert (answer["probabilities"], answer["confidence"]) == ({"only": 1.0}, 1.0)
    assert answer["action"] == {"act_probability": 0.5}  # two equal act logits


@pytest.mark.parametrize("calibrated,applied", [(0.1, 0.5), (9.0, 5.0), (2.0, 2.0)])
def test_option_count_temperature_is_clipped(calibrated, applied):
    """``temperature_by_options["<type>:<n>"]`` replaces the type's temperature for questions with
    n options, clipped to [0.5, 5]."""
    adapter = bare_adapter({"temperature": [1, 1, 1], "temperature_by_options": {"choice:2": calibrated}})
    double = {"q": {"type": "choice", "instructions": "choose", "criteria": ["a", "b"]}}
    out = adapter.decode(np.array([[0.0, 1.0]]), np.zeros((1, 2)), double, [([1, 2], [1], 0)])
    want = probabilities64([0.0, 1.0], applied)
    assert out["answers"]["q"]["probabilities"] == {"a": round(want[0], 4), "b": round(want[1], 4)}
    assert out["usage"] == {"input_tokens": 2, "output_tokens": 0}


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_nonfinite_logits_are_refused(bad):
    adapter = bare_adapter({"temperature": [1, 1, 1]})
    single = {"q": {"type": "choice", "instructions": "choose", "criteria": ["only"]}}
    with pytest.raises(RuntimeError, match="Non-finite"):
        adapter.decode(np.array([[bad]]), np.zeros((1, 2)), single, [([1, 2], [1], 0)])


def test_score_and_noul_answers():
    adapter = bare_adapter({"temperature": [1, 1, 1]})
    questions = {"s": {"type": "score", "instructions": "how", "criteria": ["low", "mid", "high"]},
                 "n": {"type": "noul", "instructions": "yes?"}}
    logits = np.array([[0.0, 0.0, 0.0], [1.0, 3.0, 0.0]], np.float32)
    out = adapter.decode(logits, np.zeros((2, 2), np.float32), questions,
                         [([1], [1], TYPES.index("score")), ([1], [1], TYPES.index("noul"))])
    s, n = out["answers"]["s"], out["answers"]["n"]
    # Uniform probabilities over three levels: expected level 1, zero confidence.
    assert s["score"] == 1.0 and s["confidence"] == 0.0
    assert s["legend"] == {"0": "low", "1": "mid", "2": "high"}
    p_true = 1 / (1 + math.exp(-2.0))  # softmax([1, 3])[1]
    assert n["noul"] == round(p_true, 4) and n["confidence"] == round(p_true, 4)
    assert list(out["answers"]) == ["s", "n"] and out["model"] == "laya-rl-agent"


def test_temperature_division_happens_in_float32():
    """16-bit logits [32, 32.03125] at temperature 0.7: the division is done in float32 (the
    reference's rounding), which is what the 4-decimal probabilities must show."""
    adapter = bare_adapter({"temperature": [0.7, 1, 1]})
    choice = {"q": {"type": "choice", "instructions": "choose", "criteria": ["a", "b"]}}
    logits = np.array([[32, 32.03125]], np.float16)
    out = adapter.decode(logits, np.zeros((1, 2), np.float16), choice, [([1, 2], [1, 2], 0)])
    scaled32 = logits[0].astype(np.float32) / np.float32(0.7)
    e = np.exp(scaled32 - scaled32.max())
    want = e / e.sum()
    assert list(out["answers"]["q"]["probabilities"].values()) == [round(float(v), 4) for v in want]


@pytest.mark.parametrize("kwargs,error,message", [
    ({"max_cached_shapes": 0}, ValueError, "max_cached_shapes"),
    ({"max_cached_shapes": 65}, ValueError, "max_cached_shapes"),
    ({"max_cached_shapes": True}, ValueError, "max_cached_shapes"),
    ({"backend": "official"}, ValueError, "backend"),
    ({"device": "cpu"}, ValueError, "device"),
])
def test_engine_argument_validation(tmp_path, kwargs, error, message):
    from laya_cuda import Engine
    with pytest.raises(error, match=message):
        Engine(tmp_path, **kwargs)


def test_checkpoint_resolution_errors(tmp_path):
    from laya_cuda.models import resolve
    with pytest.raises(FileNotFoundError, match="Incomplete checkpoint"):
        resolve(tmp_path)  # a directory without the checkpoint files
    with pytest.raises(FileNotFoundError, match="Unknown alias"):
        resolve(tmp_path / "nowhere")


def test_hosted_alias_is_not_downloaded(tmp_path):
    from laya_cuda.models import resolve
    registry = tmp_path / "models.json"
    registry.write_text(json.dumps({"hosted": {"repo_id": "org/model", "revision": "abc"}}))
    with pytest.raises(FileNotFoundError, match="does not fetch"):
        resolve("hosted", registry=registry)
    registry.write_text(json.dumps({"bad": {"path": ""}}))
    with pytest.raises(ValueError, match="Invalid model entry"):
        resolve("bad", registry=registry)


@pytest.mark.parametrize("model_type,activation", [("gpt2", "gelu"), ("modernbert", "relu"), ("bert", "silu")])
def test_unsupported_encoders_are_refused(model_type, activation):
    config = {"model_type": model_type, "hidden_size": 128, "num_attention_heads": 2, "num_hidden_layers": 1,
              "intermediate_size": 256, "vocab_size": 100, "max_position_embeddings": 128,
              "hidden_activation": activation, "hidden_act": activation}
    with pytest.raises(ValueError, match="ModernBERT"):
        Laya.from_configs(config, {"max_len": 64, "head_max_len": 32, "head_layers": 1})


def test_state_must_be_json_serialisable(tmp_path):
    from laya_cuda import synthetic
    path, _, _ = synthetic.checkpoint(tmp_path, synthetic.encoder_config(1, 64, 1, 128, 512, 128),
                                      synthetic.task_config(64))
    adapter = Laya(path)
    questions = {"q": {"type": "noul", "instructions": "yes?"}}
    assert adapter.prepare({"fine": [1, "two", None]}, questions)  # JSON values are encoded
    with pytest.raises(TypeError):
        adapter.prepare({"unsupported": object()}, questions)


def test_weight_table_of_both_variants():
    from laya_cuda import synthetic
    bert = synthetic.adapter("l512")
    shapes = bert.weight_shapes()
    assert shapes["encoder.layers.11.mlp.Wi.weight"] == (3072, 768)
    assert shapes["encoder.embeddings.position_embeddings.weight"] == (512, 768)
    assert shapes["act_head.0.weight"] == (256, 772) and shapes["act_head.2.bias"] == (2,)
    modern = Laya.from_configs({"model_type": "modernbert", "hidden_size": 768, "num_attention_heads": 12,
                                "num_hidden_layers": 3, "intermediate_size": 1152, "vocab_size": 100,
                                "max_position_embeddings": 1024},
                               {"max_len": 512, "head_max_len": 128, "head_layers": 1, "act_costs": {"x": 1}})
    m = modern.weight_shapes()
    assert m["encoder.layers.0.mlp.Wi.weight"] == (2304, 768) and "encoder.layers.0.attn_norm.weight" not in m
    assert m["encoder.layers.1.attn_norm.weight"] == (768,) and m["head.layers.0.linear1.weight"] == (3072, 768)
    assert modern.window == 64 and modern.theta == [160000.0, 10000.0]
    with pytest.raises(ValueError, match="64-wide"):
        Laya.from_configs({"model_type": "bert", "hidden_size": 768, "num_attention_heads": 8, "num_hidden_layers": 1,
                           "intermediate_size": 1, "vocab_size": 1, "max_position_embeddings": 512},
                          {"max_len": 512, "head_max_len": 1, "head_layers": 0})
