"""Laya.prepare against the reference's own outputs: token ids, option markers and kinds that the
reference's ``Laya.prepare`` (laya_cuda/laya.py:104-135) produced on the same inputs and the same
tokenizer (``tests/golden/prepare_vectors.json``, written by ``tests/golden/make_prepare_golden.py``
from the committed ``prepare_tokenizer.json``), including the ValueError it raised.  The cases
cover the three question types and their criteria forms, option, head and state truncation, the
option-budget cap, mask text, a JSON state, batched encoding, unicode and a long state (which this
build encodes in pieces)."""
import json
import shutil
from pathlib import Path

import pytest

from laya_cuda import synthetic
from laya_cuda.laya import Laya

GOLDEN = Path(__file__).resolve().parent / "golden"
VECTORS = json.loads((GOLDEN / "prepare_vectors.json").read_text(encoding="utf-8"))


def checkpoint_dir(root, max_len, head_max_len):
    root = Path(root)
    (root / "tokenizer").mkdir(parents=True)
    (root / "encoder").mkdir()
    shutil.copy(GOLDEN / VECTORS["tokenizer"], root / "tokenizer" / "tokenizer.json")
    (root / "tokenizer" / "special_tokens_map.json").write_text(json.dumps(
        {"cls_token": "[CLS]", "sep_token": "[SEP]", "mask_token": "[MASK]", "pad_token": "[PAD]"}))
    config = synthetic.modernbert_config(2, 64, 1, 128, 512, 1024, global_every=3, local_attention=64)
    (root / "encoder" / "config.json").write_text(json.dumps(config))
    (root / "rl_agent_config.json").write_text(json.dumps(
        {"max_len": max_len, "head_max_len": head_max_len, "head_layers": 1, "act_costs": {"defer": 0.05},
         "temperature": [1.0, 0.7, 1.3]}))
    return root


@pytest.fixture(scope="module")
def adapters(tmp_path_factory):
    return {tuple(b): Laya(checkpoint_dir(tmp_path_factory.mktemp(f"b{b[0]}"), *b)) for b in VECTORS["budgets"]}


@pytest.mark.parametrize("case", VECTORS["cases"], ids=lambda c: f"{c['max_len']}-{c['name']}")
def test_prepare_matches_reference_vectors(adapters, case):
    laya = adapters[(case["max_len"], case["head_max_len"])]
    if "error" in case:
        with pytest.raises(ValueError) as raised:
            laya.prepare(case["state"], case["questions"])
        assert str(raised.value) == case["error"]
        return
    got = [[list(map(int, ids)), list(map(int, markers)), int(kind)]
           for ids, markers, kind in laya.prepare(case["state"], case["questions"])]
    assert got == case["items"]


def test_vectors_exercise_the_piecewise_state_encoding(adapters):
    """The long-state cases go through the pieces path (the tokenizer splits at spaces)."""
    laya = adapters[(512, 160)]
    assert laya.prefix_cut
    long = [c for c in VECTORS["cases"] if c["name"] == "long state"]
    assert long and all(len(c["state"]) > 6 * c["max_len"] for c in long)


def test_fingerprint_is_sha256_of_compact_json(adapters):
    """input_sha256 (laya.py:192-193): sha256 of json.dumps(items, separators=(",", ":")), for the
    prepared items of every golden case and for random items."""
    import hashlib
    import random
    laya = adapters[(512, 160)]
    rng = random.Random(5)
    samples = [[(c["items"][0][0], c["items"][0][1], c["items"][0][2])] for c in VECTORS["cases"] if "items" in c]
    samples += [[([rng.randrange(0, 50000) for _ in range(rng.randrange(1, 600))],
                  sorted(rng.sample(range(1, 600), rng.randrange(1, 9))), rng.randrange(3))
                 for _ in range(rng.randrange(1, 5))] for _ in range(50)]
    for items in samples:
        want = hashlib.sha256(json.dumps(items, separators=(",", ":")).encode()).hexdigest()
        assert laya.fingerprint(items) == want
