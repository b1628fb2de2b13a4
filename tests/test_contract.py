"""Host contract (no GPU): light import, question parsing, decoding KATs, errors.

Known-answer tests are the reference's (tests/test_contract.py:11-94), applied to this package.
"""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from laya_cuda.laya import Laya, question, softmax

ROOT = Path(__file__).resolve().parents[1]


def test_import_is_light():
    subprocess.run([sys.executable, "-c", f"""
import sys
sys.path.insert(0, {str(ROOT / 'laya-cuda_amd')!r})
import laya_cuda
assert not {{'torch', 'transformers', 'cupy', 'psutil', 'pyarrow'}} & sys.modules.keys()
assert set(laya_cuda.__all__) == {{'Engine', 'BatchEngine'}}
"""], check=True)


def test_native_sources_are_ascii():
    for path in (ROOT / "laya-cuda_amd" / "csrc").glob("*.[hc]*"):
        assert path.read_bytes().isascii(), path
    assert (ROOT / "include" / "laya_hip.h").read_bytes().isascii()


def test_questions():
    q = question({"type": "choice", "instructions": {"ask": "team"}, "criteria": {"no": False, "zero": 0, "empty": None}})
    assert q[3] == ["no: false", "zero: 0", "empty"]
    assert question({"type": "noul", "instructions": "yes?"})[3] == ["false: no, the statement does not hold",
                                                                    "true: yes, the statement holds"]
    assert question({"type": "score", "instructions": "x", "criteria": ["low", {"a": 1}]})[3] == [
        "level 0: low", 'level 1: {"a": 1}']
    assert question({"type": "choice", "instructions": ["a"], "criteria": ["x"]})[1] == '["a"]'
    with pytest.raises(ValueError):
        question({"type": "choice", "instructions": "x", "criteria": []})
    with pytest.raises(ValueError, match="Unsupported question type"):
        question({"type": "rank", "instructions": "x"})
    with pytest.raises(ValueError, match="Score criteria"):
        question({"type": "score", "instructions": "x", "criteria": {"a": 1}})


def test_softmax_stable():
    np.testing.assert_allclose(softmax([10000, 10000]), [.5, .5])


def _adapter(cfg):
    adapter = object.__new__(Laya)
    adapter.cfg = cfg
    return adapter


def test_decoding_single_option_calibration_and_nonfinite():
    adapter = _adapter({"temperature": [1, 1, 1], "temperature_by_options": {"choice:2": .1}})
    single = {"q": {"type": "choice", "instructions": "choose", "criteria": ["only"]}}
    items = [([1, 2], [1], 0)]
    answer = adapter.decode(np.array([[7.]]), np.array([[0., 0.]]), single, items)["answers"]["q"]
    assert answer["probabilities"] == {"only": 1.0} and answer["confidence"] == 1.0
    assert answer["action"] == {"act_probability": .5}
    double = {"q": {"type": "choice", "instructions": "choose", "criteria": ["a", "b"]}}
    output = adapter.decode(np.array([[0., 1.]]), np.array([[0., 0.]]), double, items)
    # the calibrated temperature .1 is clipped to .5
    assert output["answers"]["q"]["probabilities"]["b"] == round(float(softmax([0, 2])[1]), 4)
    assert output["usage"] == {"input_tokens": 2, "output_tokens": 0}
    with pytest.raises(RuntimeError, match="Non-finite"):
        adapter.decode(np.array([[np.nan]]), np.array([[0., 0.]]), single, items)


def test_decode_score_and_noul_structure():
    adapter = _adapter({"temperature": [1, 1, 1]})
    questions = {"s": {"type": "score", "instructions": "how", "criteria": ["low", "mid", "high"]},
                 "n": {"type": "noul", "instructions": "yes?"}}
    logits = np.array([[0., 0., 0.], [1., 3., 0.]], np.float32)
    out = adapter.decode(logits, np.zeros((2, 2), np.float32), questions, [([1], [1], 1), ([1], [1], 2)])
    s, n = out["answers"]["s"], out["answers"]["n"]
    assert s["score"] == 1.0 and s["legend"] == {"0": "low", "1": "mid", "2": "high"} and s["confidence"] == 0.0
    p = softmax([1., 3.])
    assert n["noul"] == round(float(p[1]), 4) and n["confidence"] == round(float(max(p)), 4)
    assert list(out["answers"]) == ["s", "n"] and out["model"] == "laya-rl-agent"


def test_temperature_division_uses_fp32():
    adapter = _adapter({"temperature": [.7, 1, 1]})
    queries = {"q": {"type": "choice", "instructions": "choose", "criteria": ["a", "b"]}}
    logits = np.array([[32, 32.03125]], np.float16)
    result = adapter.decode(logits, np.array([[0, 0]], np.float16), queries, [([1, 2], [1, 2], 0)])
    expected = softmax(logits[0].astype(np.float32) / np.float32(.7))
    assert list(result["answers"]["q"]["probabilities"].values()) == [round(float(p), 4) for p in expected]


def test_missing_checkpoint_and_invalid_cache(tmp_path):
    from laya_cuda import Engine
    from laya_cuda.models import resolve
    with pytest.raises(FileNotFoundError, match="Incomplete checkpoint"):
        resolve(tmp_path)
    with pytest.raises(FileNotFoundError, match="Unknown alias"):
        resolve(tmp_path / "missing")
    for limit in (0, 65, True):
        with pytest.raises(ValueError, match="max_cached_shapes"):
            Engine(tmp_path, max_cached_shapes=limit)
    with pytest.raises(ValueError, match="backend"):
        Engine(tmp_path, backend="official")
    with pytest.raises(ValueError, match="device"):
        Engine(tmp_path, device="cpu")


def test_hosted_alias_is_not_downloaded(tmp_path):
    import json
    from laya_cuda.models import resolve
    registry = tmp_path / "models.json"
    registry.write_text(json.dumps({"hosted": {"repo_id": "org/model", "revision": "abc"}}))
    with pytest.raises(FileNotFoundError, match="does not fetch"):
        resolve("hosted", registry=registry)
    registry.write_text(json.dumps({"bad": {"path": ""}}))
    with pytest.raises(ValueError, match="Invalid model entry"):
        resolve("bad", registry=registry)


def test_unsupported_encoder_config(monkeypatch, tmp_path):
    import laya_cuda.laya as implementation
    monkeypatch.setattr(implementation, "read_json", lambda _: {"model_type": "gpt2"})
    with pytest.raises(ValueError, match="ModernBERT"):
        Laya(tmp_path)


def test_state_requires_json_values():
    adapter = object.__new__(Laya)
    adapter.tokenizer, adapter.mask_text = object(), "[MASK]"
    with pytest.raises(TypeError):
        adapter.prepare({"unsupported": object()}, {"q": {"type": "noul", "instructions": "yes?"}})


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
