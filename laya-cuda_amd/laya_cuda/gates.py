"""Accuracy gates: does a candidate inference path answer like a reference path?

The reference gates its CUDA runtime against the official SDK at FP32 (benchmarks/run.py:23,
168-203): over the same requests, the mean absolute difference of every answer probability (and
of every act probability) must be at most 1e-3, the largest at most 1e-2, and at least 99.5% of
decisions must agree.  The thresholds are the reference's; the comparison is restated here over
answer dicts as Engine.predict returns them (laya.py:137-165), request by request.

A decision is what a caller acts on: the chosen key of a choice question, whether a noul
probability reaches 0.5, and the most probable level of a score question.
"""
import math

GATES = {"probability_mae": 1e-3, "probability_max": 1e-2, "agreement": 0.995}


def decision(answer):
    kind = answer["type"]
    if kind == "choice":
        return answer["choice"]
    if kind == "noul":
        return answer["noul"] >= 0.5
    levels = answer["probabilities"]
    return max(levels, key=levels.get)


def probability_vector(answer):
    if "probabilities" in answer:
        return list(answer["probabilities"].values())
    return [1.0 - answer["noul"], answer["noul"]]


def agreement(candidates, references):
    """Statistics over aligned lists of answer dicts (one per request)."""
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
    return {"decisions": total, "agreement": same / total if total else None,
            "probability_mae": sum(diffs) / len(diffs) if diffs else None,
            "probability_max": max(diffs) if diffs else None,
            "action_mae": sum(act_diffs) / len(act_diffs) if act_diffs else None,
            "action_max": max(act_diffs) if act_diffs else None, "finite": finite}


def failures(stats, gates=GATES):
    """Names of the gates `stats` fails (empty: every gate passes)."""
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
    return failed


def passes(stats, gates=GATES):
    return not failures(stats, gates)
