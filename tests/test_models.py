"""Registry resolution (tests/test_models.py of the reference, without the hosted-download case:
this build never fetches checkpoints; tests/test_contract.py checks that refusal)."""
import json

import pytest

from laya_cuda.models import resolve


@pytest.fixture
def checkpoint(tmp_path):
    path = tmp_path / "weights"
    for name in ("model.safetensors", "rl_agent_config.json", "encoder/config.json", "tokenizer/tokenizer.json"):
        target = path / name
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text("{}")
    return path


def test_external_registry_paths(checkpoint, tmp_path, monkeypatch):
    config = tmp_path / "models.json"
    config.write_text(json.dumps({"custom": {"path": "weights"}}))
    monkeypatch.chdir(tmp_path.parent)
    assert resolve("custom", registry=config) == checkpoint
    assert resolve(checkpoint) == checkpoint


def test_local_override_of_a_builtin_alias(checkpoint, tmp_path):
    config = tmp_path / "models.json"
    config.write_text(json.dumps({"laya": {"path": "weights"}}))
    assert resolve("laya", registry=config) == checkpoint


@pytest.mark.parametrize("data", [[], {"bad": {}}, {"bad": {"repo_id": "repo"}},
    {"bad": {"path": " "}}, {"bad": {"path": 1}}, {"": {"path": "weights"}},
    {"bad": {"path": "weights", "repo_id": "repo", "revision": "rev"}}])
def test_invalid_registry(tmp_path, data):
    config = tmp_path / "models.json"
    config.write_text(json.dumps(data))
    with pytest.raises(ValueError, match="registry|entry"):
        resolve("bad", registry=config)


def test_registry_errors(tmp_path):
    config = tmp_path / "models.json"
    with pytest.raises(FileNotFoundError):
        resolve("custom", registry=config)
    config.write_text("not JSON")
    with pytest.raises(json.JSONDecodeError):
        resolve("custom", registry=config)
    config.write_text(json.dumps({"custom": {"path": "missing"}}))
    with pytest.raises(FileNotFoundError, match="Incomplete checkpoint"):
        resolve("custom", registry=config)
    with pytest.raises(FileNotFoundError, match="Unknown alias"):
        resolve("unknown", registry=config)
