"""Writes tests/golden/typed_decisions.json.gz from the reference's fixed quality fixture.

Source: benchmarks/data/typed-decisions.parquet of laya-cuda, the 400-row test split of the
LocalLLaMA/typed-decisions dataset (configuration ``all``, revision
ea9306458d6e9563628369a3d1e72e362fb381d2, Apache-2.0; attribution: LocalLLaMA, Typed Decisions
dataset).  The reference runs these 400 requests (2,000 typed decisions) through
``Engine.predict`` for its accuracy gates (benchmarks/run.py:152-160, 205-225).

Kept per row: ``id``, ``workflow``, ``state`` and ``questions`` (the JSON texts the reference's
worker passes through ``json.loads`` to ``Engine.predict``) and the gold label of each question
(``gold[qid]["label"]``, what benchmarks/run.py:184-197 compares against).  The provenance
(dataset, revision, licence, SHA-256 of the parquet file) travels in the JSON header.

Run in a container that holds the reference (pyarrow reads the parquet file; nothing of the
reference is imported):  python tests/golden/make_typed_decisions.py
"""
import gzip
import hashlib
import json
from pathlib import Path

SOURCE = Path("/root/reference/benchmarks/data/typed-decisions.parquet")
OUT = Path(__file__).resolve().parent / "typed_decisions.json.gz"


def main():
    import pyarrow.parquet as pq
    raw = SOURCE.read_bytes()
    rows = pq.read_table(SOURCE).to_pylist()
    records = [{"id": r["id"], "workflow": r["workflow"], "state": r["state"], "questions": r["questions"],
                "gold": {q: g["label"] for q, g in json.loads(r["gold"]).items()}} for r in rows]
    payload = {
        "source": "LocalLLaMA/typed-decisions, configuration all, test split, revision "
                  "ea9306458d6e9563628369a3d1e72e362fb381d2 (via laya-cuda benchmarks/data/typed-decisions.parquet)",
        "license": "Apache-2.0; attribution: LocalLLaMA, Typed Decisions dataset; labels are synthetic pseudo-labels",
        "parquet_sha256": hashlib.sha256(raw).hexdigest(),
        "records": records,
    }
    data = json.dumps(payload, ensure_ascii=False, separators=(",", ":")).encode()
    with gzip.GzipFile(OUT, "wb", compresslevel=9, mtime=0) as f:
        f.write(data)
    print(f"{len(records)} requests, {sum(len(r['gold']) for r in records)} decisions -> {OUT} "
          f"({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
