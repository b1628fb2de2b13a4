"""Write token-layout golden vectors of the reference's ``Laya.prepare`` (laya_cuda/laya.py:104-135).

Run once in a container that has the reference sources at /root/reference (never during the tests,
never on the GPU host):  python tests/golden/make_prepare_golden.py

``Laya.prepare`` is host code that no other check pins at the level of token ids: the reference's
own tests of it need a hosted checkpoint.  This script imports the reference's ``laya.py`` (and
the ``models.py`` it imports ``read_json`` from) straight from its files, without its package
``__init__`` (which imports the CUDA runtime), builds ``Laya`` on checkpoint directories whose
tokenizer is this repository's offline-trained byte-pair tokenizer (``prepare_tokenizer.json``,
committed beside this script), and records ``prepare``'s output - ids, option markers, kinds - or the
ValueError message for each case.  ``tests/test_prepare_golden.py`` compares this build's
``Laya.prepare`` with the vectors.
"""
import importlib.util
import json
import sys
import tempfile
import types
from pathlib import Path

REFERENCE = Path("/root/reference/laya_cuda")
HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "laya-cuda_amd"))
from laya_cuda import synthetic  # noqa: E402

TOKENIZER = HERE / "prepare_tokenizer.json"
OUT = HERE / "prepare_vectors.json"

# Budgets (max_len, head_max_len) of the two checkpoint directories.
BUDGETS = [(128, 48), (512, 160)]

LONG_STATE = " ".join(["the customer asks about a late delivery and wants a refund for order", str(n),
                       "billing team handles invoices; shipping team handles tracking."][i % 3]
                      for n in range(70) for i in range(3))


def cases():
    """(name, state, questions) covering every branch of prepare: the three question types and
    their criteria forms, option and head truncation, the option-budget cap, state truncation,
    mask text in any field, a JSON state, batched encoding (12+ texts) and the budget error."""
    route = {"type": "choice", "instructions": "Choose a team for the ticket",
             "criteria": {"billing": "invoices and payment errors", "shipping": "delivery and tracking",
                          "other": None, "software": ""}}
    urgency = {"type": "score", "instructions": "How urgent is the ticket?",
               "criteria": ["not urgent", "urgent", {"level": "critical", "pager": True}]}
    angry = {"type": "noul", "instructions": "Is the customer angry?"}
    angry_custom = {"type": "noul", "instructions": {"ask": "angry?"}, "criteria": {"true": "very angry", "false": ""}}
    listed = {"type": "choice", "instructions": "Choose a topic", "criteria": ["billing", "shipping", "other"]}
    many = {"type": "choice", "instructions": "Route the ticket to the right queue",
            "criteria": {f"queue {i}": "software questions go to the engineering queue " * 3 for i in range(12)}}
    long_option = {"type": "choice", "instructions": "Choose",
                   "criteria": {"a": "refund the payment for the order " * 20, "b": "level 1: urgent"}}
    long_head = {"type": "score", "instructions": "the customer asks about a late delivery " * 30,
                 "criteria": ["low", "high"]}
    masked = {"type": "choice", "instructions": "Choose [MASK] team",
              "criteria": {"billing [MASK]": "payment [MASK] errors", "other": None}}
    too_many = {"type": "choice", "instructions": "Choose",
                "criteria": {f"option {i}": None for i in range(200)}}
    yield "short choice", "refund the payment for the order", {"route": route}
    yield "three types", "the customer asks about a late delivery and wants a refund", {
        "route": route, "urgency": urgency, "angry": angry}
    yield "listed criteria and custom noul", "payment software ticket", {"topic": listed, "angry": angry_custom}
    yield "empty state", "", {"route": route}
    yield "long state", LONG_STATE, {"route": route, "angry": angry}
    yield "json state", {"ticket": 17, "text": "late delivery", "tags": ["billing", "urgent"], "note": "[MASK]"}, {
        "urgency": urgency}
    yield "option budget cap", "customer delivery", {"many": many}
    yield "long option", LONG_STATE[:900], {"long": long_option}
    yield "long head", "order", {"head": long_head}
    yield "mask text", "the [MASK] customer asks about a [MASK]refund", {"masked": masked}
    yield "batched encode", LONG_STATE[:3000], {f"q{i}": (route if i % 2 else urgency) for i in range(4)}
    yield "unicode", "Café délai de livraison — 配送が遅れています 😀 refund", {"angry": angry, "route": route}
    yield "budget error", "refund", {"too_many": too_many}


def load_reference():
    """The reference's models.py and laya.py as modules of a stand-in package (its __init__, which
    imports the CUDA engine, is not run)."""
    package = types.ModuleType("laya_reference")
    package.__path__ = [str(REFERENCE)]
    sys.modules["laya_reference"] = package
    modules = {}
    for name in ("models", "laya"):
        spec = importlib.util.spec_from_file_location(f"laya_reference.{name}", REFERENCE / f"{name}.py")
        module = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = module
        spec.loader.exec_module(module)
        modules[name] = module
    return modules["laya"]


def checkpoint_dir(root, max_len, head_max_len):
    """Configs and tokenizer of a ModernBERT Laya checkpoint (prepare reads no weights)."""
    root = Path(root)
    (root / "tokenizer").mkdir(parents=True)
    (root / "encoder").mkdir()
    (root / "tokenizer" / "tokenizer.json").write_text(TOKENIZER.read_text(encoding="utf-8"), encoding="utf-8")
    (root / "tokenizer" / "special_tokens_map.json").write_text(json.dumps(
        {"cls_token": "[CLS]", "sep_token": "[SEP]", "mask_token": "[MASK]", "pad_token": "[PAD]"}))
    config = synthetic.modernbert_config(2, 64, 1, 128, 512, 1024, global_every=3, local_attention=64)
    (root / "encoder" / "config.json").write_text(json.dumps(config))
    task = {"max_len": max_len, "head_max_len": head_max_len, "head_layers": 1, "act_costs": {"defer": 0.05},
            "temperature": [1.0, 0.7, 1.3]}
    (root / "rl_agent_config.json").write_text(json.dumps(task))
    return root


def main():
    if not TOKENIZER.is_file():
        synthetic.tokenizer().save(str(TOKENIZER))
    reference = load_reference()
    out = {"tokenizer": TOKENIZER.name, "budgets": BUDGETS, "cases": []}
    with tempfile.TemporaryDirectory() as tmp:
        for max_len, head_max_len in BUDGETS:
            laya = reference.Laya(checkpoint_dir(Path(tmp) / f"b{max_len}", max_len, head_max_len))
            for name, state, questions in cases():
                entry = {"name": name, "max_len": max_len, "head_max_len": head_max_len, "state": state,
                         "questions": questions}
                try:
                    entry["items"] = [[list(map(int, ids)), list(map(int, markers)), int(kind)]
                                      for ids, markers, kind in laya.prepare(state, questions)]
                except ValueError as error:
                    entry["error"] = str(error)
                out["cases"].append(entry)
    OUT.write_text(json.dumps(out, ensure_ascii=False, indent=0) + "\n", encoding="utf-8")
    print(f"wrote {OUT} ({len(out['cases'])} cases)")


if __name__ == "__main__":
    main()
