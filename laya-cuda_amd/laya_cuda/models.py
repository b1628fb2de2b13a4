"""JSON checkpoint configuration and a small model adapter registry (laya_cuda/models.py:1-58).

Local directories and ``{"path": ...}`` registry entries resolve as in the reference.  Entries
pinned to a hosted ``repo_id``/``revision`` need a network download, which this build does not
perform: they raise with a message naming the entry.
"""
import json
from pathlib import Path

FILES = ["model.safetensors", "rl_agent_config.json", "encoder/config.json", "tokenizer/*"]


def read_json(path):
    return json.loads(Path(path).read_text(encoding="utf-8"))


def _checkpoints(registry=None):
    sources = [Path(__file__).with_name("models.json")]
    if registry is not None:
        sources.append(Path(registry).expanduser())
    entries = {}
    for source in sources:
        if not source.is_file():
            continue
        data = read_json(source)
        if not isinstance(data, dict):
            raise ValueError(f"Model registry must be a JSON object: {source}")
        for alias, entry in data.items():
            valid = (alias.strip() and isinstance(entry, dict)
                     and set(entry) in ({"path"}, {"repo_id", "revision"})
                     and all(isinstance(v, str) and v.strip() for v in entry.values()))
            if not valid:
                raise ValueError(f"Invalid model entry {alias!r} in {source}; use path or repo_id and revision")
            if "path" in entry:
                entry = {"path": str((source.parent / Path(entry["path"]).expanduser()).resolve())}
            entries[alias] = entry
    return entries


def resolve(model, revision=None, *, registry=None):
    """Local checkpoint directory for ``model`` (a path or a registry alias)."""
    path = Path(model).expanduser()
    if not path.is_dir():
        checkpoints = _checkpoints(registry)
        if str(model) not in checkpoints:
            raise FileNotFoundError(f"Unknown alias or missing local checkpoint: {model}")
        entry = checkpoints[str(model)]
        if "path" not in entry:
            raise FileNotFoundError(
                f"Alias {model!r} names hosted checkpoint {entry['repo_id']}@{revision or entry['revision']}; "
                "download it and pass the local directory (this runtime does not fetch checkpoints)")
        path = Path(entry["path"])
    for name in FILES[:3] + ["tokenizer/tokenizer.json"]:
        if not (path / name).is_file():
            raise FileNotFoundError(f"Incomplete checkpoint: {path / name}")
    return path.resolve()


def adapter(path):
    from .laya import Laya
    registry = {"laya": Laya}
    kind = "laya" if (path / "rl_agent_config.json").is_file() else None
    if kind not in registry:
        raise ValueError("No compatible model adapter")
    return registry[kind](path)
