"""Accuracy gates: does a candidate inference path answer like a reference path?

The reference gates its CUDA runtime against the official SDK at FP32 (benchmarks/run.py:23,
168-225): over the same requests, the mean absolute difference of every answer probability (and
of every act probability) must be at most 1e-3, the largest at most 1e-2, at least 99.5% of
decisions must agree, and - where the requests carry gold labels - the candidate's accuracy may
not fall significantly below the reference's: an exact one-sided sign test over the decisions
exactly one side gets right must give p >= 0.05 (run.py:184-197, applied at :220).  The
thresholds are the reference's; the comparison is restated here over answer dicts as
Engine.predict returns them (laya.py:137-165), request by request.

A decision is what a caller acts on: the chosen key of a choice question, "true" or "false" as a
noul probability reaches 0.5 or not, and the most probable level of a score question (the label
strings gold labels use).
"""
import math

GATES = {"probability_mae": 1e-3, "probability_max": 1e-2, "agreement": 0.995, "accuracy_sign_test_p": 0.05}


def decision(answer):
    kind = answer["type"]
    if kind == "choice":
        return answer["choice"]
    if kind == "noul":
        return "true" if answer["noul"] >= 0.5 else "false"
    levels = answer["probabilities"]
    return max(levels, key=levels.get)


def probability_vector(answer):
    if "probabilities" in answer:
        return list(answer["probabilities"].values())
    return [1.0 - answer["noul"], answer["noul"]]


def sign_test(wins, losses):
    """One-sided exact sign test: the probability that a fair coin over the wins + losses decisions
    only one side gets right gives at least `losses` losses, sum_{k >= losses} C(n, k) / 2^n."""
    n = wins + losses
    if not n:
        return 1.0
    return sum(math.comb(n, k) for k in range(losses, n + 1)) / 2 ** n


def accuracy_test(candidates, references, gold):
    """Wins (candidate right, reference wrong) and losses (the reverse) against gold labels, and the
    sign test's p-value.  ``gold``: one {question id: label} dict per request."""
    if not len(candidates) == len(references) == len(gold):
        raise ValueError("candidate, reference and gold lists differ in length")
    wins = losses = right_c = right_r = total = 0
    for got, want, labels in zip(candidates, references, gold):
        for qid, label in labels.items():
            a = decision(got["answers"][qid]) == str(label)
            b = decision(want["answers"][qid]) == str(label)
            wins += a and not b
            losses += b and not a
            right_c += a
            right_r += b
            total += 1
    return {"wins": wins, "losses": losses, "p_value": sign_test(wins, losses),
            "accuracy": right_c / total if total else None, "reference_accuracy": right_r / total if total else None}


def agreement(candidates, references, gold=None):
    """Statistics over aligned lists of answer dicts (one per request); with ``gold`` (one
    {question id: label} dict per request) also the accuracy sign test."""
    if len(candidates) != len(references):
        raise ValueError("candidate and reference answer lists differ in length")
    diffs, act_diffs, same, total = [], [], 0, 0
    for got, want in zip(candidates, references):
        if list(got["answers"]) != list(want["answers"]):
            raise ValueError("candidate and reference answer different questions")
        for qid, a in got["answers"].items():
            b = want["answers"][qid]
            pa, pb = probability_vector(a), probability_vector(b)
            if len(pa) != len(pb):
                raise ValueError(f"question {qid!r}: option counts differ")
            diffs.extend(abs(x - y) for x, y in zip(pa, pb))
            act_diffs.append(abs(a["action"]["act_probability"] - b["action"]["act_probability"]))
            same += decision(a) == decision(b)
            total += 1
    finite = all(math.isfinite(v) for v in diffs + act_diffs)
    stats = {"decisions": total, "agreement": same / total if total else None,
             "probability_mae": sum(diffs) / len(diffs) if diffs else None,
             "probability_max": max(diffs) if diffs else None,
             "action_mae": sum(act_diffs) / len(act_diffs) if act_diffs else None,
             "action_max": max(act_diffs) if act_diffs else None, "finite": finite}
    if gold is not None:
        stats["accuracy_test"] = accuracy_test(candidates, references, gold)
    return stats


def failures(stats, gates=GATES):
    """Names of the gates `stats` fails (empty: every gate passes).  The accuracy sign test is a
    gate whenever the statistics carry it (requests with gold labels)."""
    if not stats["decisions"]:
        return ["no decisions"]
    if not stats["finite"]:
        return ["non-finite probabilities"]
    failed = []
    for key, limit in (("probability_mae", gates["probability_mae"]), ("action_mae", gates["probability_mae"]),
                       ("probability_max", gates["probability_max"]), ("action_max", gates["probability_max"])):
        if stats[key] > limit:
            failed.append(f"{key} {stats[key]:.3g} > {limit:g}")
    if stats["agreement"] < gates["agreement"]:
        failed.append(f"agreement {stats['agreement']:.4f} < {gates['agreement']:g}")
    test = stats.get("accuracy_test")
    if test is not None and test["p_value"] < gates["accuracy_sign_test_p"]:
        failed.append(f"accuracy sign test p {test['p_value']:.4g} < {gates['accuracy_sign_test_p']:g} "
                      f"({test['wins']} wins, {test['losses']} losses)")
    return failed


def passes(stats, gates=GATES):
    return not failures(stats, gates)
