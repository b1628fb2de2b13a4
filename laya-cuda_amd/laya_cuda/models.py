"""Checkpoint location: a local directory, or an alias that a JSON registry maps to one.

The reference resolves aliases to hosted checkpoints and downloads them (laya_cuda/models.py:
31-47).  This runtime never fetches anything: ``resolve`` accepts a checkpoint directory, or an
alias from the ``registry`` file whose entry is ``{"path": dir}`` (relative paths are taken from
the registry file's folder).  Entries naming a hosted ``repo_id``/``revision`` are recognised and
refused with a message that says so.  Error types follow the reference: ``FileNotFoundError`` for
unknown aliases and incomplete checkpoints, ``ValueError`` for a malformed registry.
"""
import json
from pathlib import Path

# Files a Laya checkpoint directory must hold (laya_cuda/models.py:6 lists them as download patterns).
REQUIRED = ("model.safetensors", "rl_agent_config.json", "encoder/config.json", "tokenizer/tokenizer.json")


def read_json(path):
    return json.loads(Path(path).read_text(encoding="utf-8"))


def _text(value):
    return isinstance(value, str) and bool(value.strip())


def _lookup(alias, registry):
    """The registry entry for ``alias`` ({"path": absolute} or {"repo_id", "revision"}), or None."""
    if registry is None:
        return None
    source = Path(registry).expanduser()
    table = read_json(source)  # FileNotFoundError / JSONDecodeError propagate
    if not isinstance(table, dict):
        raise ValueError(f"Model registry must be a JSON object: {source}")
    found = None
    for name, entry in table.items():
        local = isinstance(entry, dict) and set(entry) == {"path"}
        hosted = isinstance(entry, dict) and set(entry) == {"repo_id", "revision"}
        if not (_text(name) and (local or hosted) and all(_text(v) for v in entry.values())):
            raise ValueError(f"Invalid model entry {name!r} in {source}; use path or repo_id and revision")
        if name == alias:
            found = {"path": str((source.parent / Path(entry["path"]).expanduser()).resolve())} if local else entry
    return found


def resolve(model, revision=None, *, registry=None):
    """Absolute path of the checkpoint directory ``model`` names (a directory or a registry alias)."""
    directory = Path(model).expanduser()
    if not directory.is_dir():
        entry = _lookup(str(model), registry)
        if entry is None:
            raise FileNotFoundError(f"Unknown alias or missing local checkpoint: {model}")
        if "path" not in entry:
            raise FileNotFoundError(
                f"Alias {model!r} names hosted checkpoint {entry['repo_id']}@{revision or entry['revision']}; "
                "this runtime does not fetch checkpoints: download it and pass the local directory")
        directory = Path(entry["path"])
    missing = [name for name in REQUIRED if not (directory / name).is_file()]
    if missing:
        raise FileNotFoundError(f"Incomplete checkpoint: {directory / missing[0]}")
    return directory.resolve()


def adapter(path):
    """The model adapter for a checkpoint directory (Laya checkpoints carry rl_agent_config.json)."""
    if not (Path(path) / "rl_agent_config.json").is_file():
        raise ValueError("No compatible model adapter")
    from .laya import Laya
    return Laya(Path(path))
