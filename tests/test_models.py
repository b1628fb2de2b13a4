"""Checkpoint resolution: local directories and registry aliases, never a download (no GPU).

The contract is the reference's resolve()/adapter() (laya_cuda/models.py:31-58) minus hosted
downloads: FileNotFoundError for unknown aliases and incomplete checkpoints, ValueError for a
malformed registry, relative registry paths taken from the registry file's folder."""
import json

import pytest

from laya_cuda import models
from laya_cuda.models import REQUIRED, resolve


def make_checkpoint(root, skip=()):
    for name in REQUIRED:
        if name in skip:
            continue
        target = root / name
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text("{}")
    return root


def write_registry(path, table):
    path.write_text(json.dumps(table))
    return path


def test_directory_resolves_to_its_absolute_path(tmp_path, monkeypatch):
    ckpt = make_checkpoint(tmp_path / "ckpt")
    monkeypatch.chdir(tmp_path)
    assert resolve("ckpt") == ckpt.resolve()
    assert resolve(ckpt) == ckpt.resolve()


@pytest.mark.parametrize("missing", REQUIRED)
def test_every_required_file_is_checked(tmp_path, missing):
    ckpt = make_checkpoint(tmp_path / "ckpt", skip=(missing,))
    with pytest.raises(FileNotFoundError, match="Incomplete checkpoint") as info:
        resolve(ckpt)
    assert missing.split("/")[-1] in str(info.value)


def test_registry_alias_paths_are_relative_to_the_registry(tmp_path, monkeypatch):
    ckpt = make_checkpoint(tmp_path / "models" / "fine-tuned")
    registry = write_registry(tmp_path / "models" / "registry.json",
                              {"tuned": {"path": "fine-tuned"}, "abs": {"path": str(ckpt)}})
    monkeypatch.chdir(tmp_path.parent)  # not the registry's folder
    assert resolve("tuned", registry=registry) == ckpt.resolve()
    assert resolve("abs", registry=str(registry)) == ckpt.resolve()
    with pytest.raises(FileNotFoundError, match="Unknown alias"):
        resolve("other", registry=registry)
    with pytest.raises(FileNotFoundError, match="Unknown alias"):
        resolve("tuned")  # no registry given


def test_hosted_entries_are_refused_without_network(tmp_path, monkeypatch):
    import sys
    monkeypatch.setitem(sys.modules, "huggingface_hub", None)  # any import attempt would fail loudly
    registry = write_registry(tmp_path / "r.json", {"hub": {"repo_id": "org/laya", "revision": "r1"}})
    with pytest.raises(FileNotFoundError, match="does not fetch") as info:
        resolve("hub", registry=registry)
    assert "org/laya@r1" in str(info.value)
    with pytest.raises(FileNotFoundError, match="org/laya@pinned"):
        resolve("hub", revision="pinned", registry=registry)


@pytest.mark.parametrize("table", [
    [], "text", {"x": {}}, {"x": {"path": ""}}, {"x": {"path": 3}}, {"x": {"repo_id": "a"}},
    {" ": {"path": "p"}}, {"x": {"path": "p", "repo_id": "a", "revision": "b"}}, {"x": "p"}])
def test_malformed_registries_raise_value_error(tmp_path, table):
    registry = write_registry(tmp_path / "r.json", table)
    with pytest.raises(ValueError, match="registry|entry"):
        resolve("x", registry=registry)


def test_unreadable_registries(tmp_path):
    registry = tmp_path / "r.json"
    with pytest.raises(FileNotFoundError):
        resolve("x", registry=registry)
    registry.write_text("{not json")
    with pytest.raises(json.JSONDecodeError):
        resolve("x", registry=registry)


def test_adapter_needs_a_laya_config(tmp_path):
    with pytest.raises(ValueError, match="No compatible model adapter"):
        models.adapter(tmp_path)
