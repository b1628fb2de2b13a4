"""The reference's fixed quality fixture as requests (test infrastructure).

tests/golden/typed_decisions.json.gz holds the 400 requests (2,000 typed decisions, with gold
labels) that the reference runs through ``Engine.predict`` for its accuracy gates
(benchmarks/run.py:152-160; written by tests/golden/make_typed_decisions.py).  ``long_cases``
restates how the reference builds 48 long inputs from them (run.py:76-94): request i takes the
questions of record 7i, and the states of records i, i+13, i+26, ... joined by newlines until the
longest question's token layout reaches a target that cycles through 60%-100% of the context
budget (or 61 states are joined).
"""
import gzip
import json
from pathlib import Path

FIXTURE = Path(__file__).resolve().parent / "golden" / "typed_decisions.json.gz"


def records():
    """[{id, workflow, state, questions, gold}], ``state``/``questions`` as the JSON texts."""
    return json.loads(gzip.decompress(FIXTURE.read_bytes()))["records"]


def requests(rows=None):
    """(id, state, questions, gold labels) per record, parsed as the reference's worker does."""
    return [(r["id"], json.loads(r["state"]), json.loads(r["questions"]), r["gold"]) for r in (rows or records())]


def long_cases(adapter, rows=None, count=48):
    """(name, state text, questions, tokens) of the reference's long-input suite."""
    rows = rows or records()
    low = int(adapter.max_len * 0.6)
    out = []
    for i in range(count):
        target = low + (i * 37) % (adapter.max_len - low)
        questions = json.loads(rows[(i * 7) % len(rows)]["questions"])
        states, j = [], i
        while True:
            states.append(json.dumps(json.loads(rows[j % len(rows)]["state"]), ensure_ascii=False))
            state = "\n".join(states)
            tokens = max(len(ids) for ids, _, _ in adapter.prepare(state, questions))
            if tokens >= target or len(states) > 60:
                break
            j += 13
        out.append((f"long-{i}", state, questions, tokens))
    return out
