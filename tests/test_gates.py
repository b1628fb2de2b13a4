"""Accuracy-gate logic (benchmarks/run.py:23, 168-203 thresholds) on constructed answer dicts (no GPU).

A planted mistake in a candidate (a shifted probability, a flipped decision, a changed act
probability, a non-finite value) must fail exactly the gate it concerns."""
import copy
import math

import pytest

from laya_cuda import gates


def choice(probs, act=0.5):
    keys = [f"k{i}" for i in range(len(probs))]
    return {"type": "choice", "probabilities": dict(zip(keys, probs)), "choice": keys[probs.index(max(probs))],
            "action": {"act_probability": act}}


def noul(p, act=0.5):
    return {"type": "noul", "noul": p, "action": {"act_probability": act}}


def score(probs, act=0.5):
    return {"type": "score", "probabilities": {str(i): v for i, v in enumerate(probs)}, "action": {"act_probability": act}}


def request(*answers):
    return {"answers": {f"q{i}": a for i, a in enumerate(answers)}}


REFERENCE = [request(choice([0.6, 0.3, 0.1]), noul(0.8), score([0.2, 0.5, 0.3])) for _ in range(100)]  # 300 decisions


def test_identical_answers_pass_every_gate():
    stats = gates.agreement(REFERENCE, copy.deepcopy(REFERENCE))
    assert stats["decisions"] == 300 and stats["agreement"] == 1.0
    assert stats["probability_mae"] == 0 and stats["probability_max"] == 0 and stats["action_max"] == 0
    assert gates.passes(stats) and gates.failures(stats) == []


def test_decisions_follow_the_answer_type():
    assert gates.decision(choice([0.2, 0.7, 0.1])) == "k1"
    assert gates.decision(noul(0.5)) == "true" and gates.decision(noul(0.4999)) == "false"
    assert gates.decision(score([0.1, 0.3, 0.6])) == "2"
    assert gates.probability_vector(noul(0.25)) == [0.75, 0.25]


def test_probability_mae_and_max_gates():
    cand = copy.deepcopy(REFERENCE)
    cand[0]["answers"]["q0"]["probabilities"]["k1"] += 0.009  # max 9e-3 (< 1e-2), mean tiny
    stats = gates.agreement(cand, REFERENCE)
    assert math.isclose(stats["probability_max"], 0.009) and gates.passes(stats)
    cand[0]["answers"]["q0"]["probabilities"]["k1"] += 0.002  # max 1.1e-2
    assert gates.failures(gates.agreement(cand, REFERENCE)) == ["probability_max 0.011 > 0.01"]
    shifted = copy.deepcopy(REFERENCE)
    for r in shifted:
        r["answers"]["q2"]["probabilities"]["1"] += 0.005  # mean over 800 values: 100*0.005/800
    stats = gates.agreement(shifted, REFERENCE)
    assert math.isclose(stats["probability_mae"], 0.000625) and gates.passes(stats)
    for r in shifted:
        r["answers"]["q1"]["noul"] += 0.004  # +2 values of 0.004 per request
    stats = gates.agreement(shifted, REFERENCE)
    assert stats["probability_mae"] > 1e-3 and any(f.startswith("probability_mae") for f in gates.failures(stats))


def test_action_gates():
    cand = copy.deepcopy(REFERENCE)
    cand[3]["answers"]["q1"]["action"]["act_probability"] = 0.52
    failed = gates.failures(gates.agreement(cand, REFERENCE))
    assert failed == ["action_max 0.02 > 0.01"]


def test_agreement_gate_counts_flipped_decisions():
    cand = copy.deepcopy(REFERENCE)
    cand[7]["answers"]["q1"]["noul"] = 0.49  # one flip in 300: 0.99667 >= 0.995
    # (the probability moved by 0.31: exclude the probability gates from this check)
    stats = gates.agreement(cand, REFERENCE)
    assert math.isclose(stats["agreement"], 299 / 300)
    assert not any(f.startswith("agreement") for f in gates.failures(stats))
    cand[8]["answers"]["q0"]["choice"] = "k2"  # two flips: 0.99333 < 0.995
    stats = gates.agreement(cand, REFERENCE)
    assert any(f.startswith("agreement 0.9933") for f in gates.failures(stats))


def test_misaligned_or_non_finite_inputs():
    with pytest.raises(ValueError):
        gates.agreement(REFERENCE[:3], REFERENCE[:2])
    with pytest.raises(ValueError):
        gates.agreement([request(noul(0.5))], [request(noul(0.5), noul(0.5))])
    with pytest.raises(ValueError):
        gates.agreement([request(choice([0.5, 0.5]))], [request(choice([0.2, 0.3, 0.5]))])
    cand = copy.deepcopy(REFERENCE)
    cand[0]["answers"]["q1"]["noul"] = float("nan")
    assert gates.failures(gates.agreement(cand, REFERENCE)) == ["non-finite probabilities"]
    assert gates.failures(gates.agreement([], [])) == ["no decisions"]


@pytest.mark.parametrize("wins,losses,p", [
    (0, 0, 1.0),          # nothing decided differently
    (3, 0, 1.0),          # no losses: every outcome has at least 0
    (0, 1, 0.5),          # C(1,1)/2
    (0, 4, 1 / 16),       # C(4,4)/16
    (0, 5, 1 / 32),       # 0.03125 < 0.05
    (1, 4, 6 / 32),       # (C(5,4) + C(5,5))/32
    (2, 7, 46 / 512),     # (36 + 9 + 1)/512
    (5, 5, 638 / 1024),   # sum_{k>=5} C(10,k)/1024
])
def test_sign_test_p_values(wins, losses, p):
    assert math.isclose(gates.sign_test(wins, losses), p, rel_tol=1e-12)


def test_accuracy_gate_uses_gold_labels():
    """Candidate and reference disagree only where a gold label exists: five questions the
    reference gets right and the candidate wrong (p = 1/32) fail the accuracy gate even though
    agreement stays above 99.5%; a balanced set of disagreements passes it."""
    n = 1000
    ref = [request(choice([0.6, 0.4])) for _ in range(n)]  # decides k0
    cand = copy.deepcopy(ref)
    gold = [{} for _ in range(n)]
    for i in range(5):  # candidate flips to k1 on five gold-k0 questions (probabilities move too)
        cand[i]["answers"]["q0"] = choice([0.4, 0.6])
        gold[i]["q0"] = "k0"
    stats = gates.agreement(cand, ref, gold)
    assert stats["accuracy_test"] == {"wins": 0, "losses": 5, "p_value": 1 / 32, "accuracy": 0.0,
                                      "reference_accuracy": 1.0}
    assert stats["agreement"] == 0.995
    failed = gates.failures(stats, {**gates.GATES, "probability_max": 1.0, "probability_mae": 1.0})
    assert failed == ["accuracy sign test p 0.03125 < 0.05 (0 wins, 5 losses)"]
    for i in range(5, 8):  # three flips where the candidate is right: 3 wins, 5 losses
        cand[i]["answers"]["q0"] = choice([0.4, 0.6])
        gold[i]["q0"] = "k1"
    test = gates.agreement(cand, ref, gold)["accuracy_test"]
    assert (test["wins"], test["losses"]) == (3, 5) and math.isclose(test["p_value"], 93 / 256)
    # Without gold labels the accuracy gate does not apply.
    assert "accuracy_test" not in gates.agreement(cand, ref)
    with pytest.raises(ValueError):
        gates.accuracy_test(cand, ref, gold[:-1])
