"""The command line (python -m laya_cuda): argument errors, single and JSONL prediction with a
stand-in Engine, and the doctor's report on a machine without a usable device (no GPU)."""
import json

import pytest

import laya_cuda.engine as engine_module
from laya_cuda import cli


class StandInEngine:
    def __init__(self, model, device="cuda:0"):
        self.model, self.last_metrics = model, {"gpu_ms": 0.25}

    def predict(self, state, questions):
        if state == "boom":
            raise RuntimeError("device lost")
        return {"model": self.model, "answers": {q: {"echo": state} for q in questions}}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


@pytest.fixture
def stand_in(monkeypatch):
    monkeypatch.setattr(engine_module, "Engine", StandInEngine)


def test_usage_errors(stand_in, capsys):
    assert cli.main(["predict"]) == 2
    assert "exactly one of STATE or --input" in capsys.readouterr().err
    assert cli.main(["predict", "text"]) == 2
    assert "--questions is required" in capsys.readouterr().err
    assert cli.main(["predict", "text", "-q", "{not json"]) == 2
    assert "not valid JSON" in capsys.readouterr().err
    assert cli.main(["predict", "text", "-q", "missing.json"]) == 2
    with pytest.raises(SystemExit):
        cli.main(["frobnicate"])


def test_single_prediction(stand_in, capsys, tmp_path):
    questions = tmp_path / "q.json"
    questions.write_text(json.dumps({"topic": {"type": "noul", "instructions": "?"}}))
    assert cli.main(["predict", "hello", "-q", str(questions), "-m", "ckpt", "--metrics"]) == 0
    out = json.loads(capsys.readouterr().out)
    assert out["answers"] == {"topic": {"echo": "hello"}} and out["model"] == "ckpt" and out["metrics"]["gpu_ms"] == 0.25


def test_jsonl_lines_fail_alone(stand_in, capsys, tmp_path):
    requests = tmp_path / "r.jsonl"
    requests.write_text("\n".join([
        json.dumps({"id": "a", "state": "one"}),
        "{broken",
        json.dumps({"id": "c", "state": "boom"}),
        json.dumps({"state": "four", "questions": {"own": {}}}),
        json.dumps(["not", "an", "object"]),
        ""]))
    out_file = tmp_path / "out.jsonl"
    code = cli.main(["predict", "-i", str(requests), "-q", '{"shared": {}}', "-o", str(out_file)])
    assert code == 1 and "3 request(s) failed" in capsys.readouterr().err
    records = [json.loads(line) for line in out_file.read_text().splitlines()]
    assert [r["id"] for r in records] == ["a", 2, "c", 4, 5]
    assert records[0]["answers"] == {"shared": {"echo": "one"}}
    assert "JSONDecodeError" in records[1]["error"] and "device lost" in records[2]["error"]
    assert records[3]["answers"] == {"own": {"echo": "four"}} and "error" in records[4]


def test_doctor_without_a_device_fails_cleanly(capsys):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: tests/test_doctor_gpu.py covers the doctor there")
    assert cli.main(["doctor", "--json"]) == 1
    report = json.loads(capsys.readouterr().out)
    assert not report["passed"]
    checks = {c["check"]: c["status"] for c in report["checks"]}
    assert checks["library"] == "ok" and checks["devices"] == "fail"
    assert cli.main(["doctor", "--device", "gpu0"]) == 1
    assert "device must be" in capsys.readouterr().out
