"""BatchEngine scheduling, budgets and failure routing, driven from the host by a scripted stand-in
for Engine (no GPU).  Behaviour under test is the reference's BatchEngine contract
(laya_cuda/batching.py:17-157): one device-owning thread, input snapshots at submission,
arrival-order packing within the question and packed-row budgets, per-request errors, bounded
queue, cancellation, drain on close, and a fatal worker error reaching every waiter.
"""
from concurrent.futures import ThreadPoolExecutor, wait
from queue import Full
import threading

import pytest

import laya_cuda.batching as batching
from laya_cuda import BatchEngine


class Script:
    """A stand-in for Engine.  A request's state is {"tag": str, "rows": [token counts...]} plus
    optional "fail" in {"prepare", "predict", "decode", "fatal"}; questions map ids to anything.
    prepare() yields one item per token count; predict() records the pack's tags; decode() answers
    {question id: tag}."""

    def __init__(self):
        self.packs, self.threads = [], set()
        self.gate = threading.Event()
        self.gate.set()
        self.busy = threading.Event()
        self.closed = 0

    def install(self, monkeypatch):
        script = self

        class StandIn:
            def __init__(self, *args, **kwargs):
                script.threads.add(threading.get_ident())
                self.adapter = self.runtime = self

            def prepare(self, state, questions):
                script.threads.add(threading.get_ident())
                if state.get("fail") == "prepare" or not questions:
                    raise ValueError(f"cannot prepare {state['tag']}")
                return [([0] * n, [1], 0, state) for n in state["rows"]]

            def predict(self, items):
                script.threads.add(threading.get_ident())
                script.busy.set()
                assert script.gate.wait(10)
                tags = []
                for item in items:
                    if item[3]["tag"] not in tags:
                        tags.append(item[3]["tag"])
                script.packs.append(tags)
                modes = {item[3].get("fail") for item in items}
                if "fatal" in modes:
                    raise SystemExit("owner thread stopped")
                if "predict" in modes:
                    raise RuntimeError("device lost")
                return [item[3]["tag"] for item in items], [0.0] * len(items), {"gpu_ms": 0.5}

            def decode(self, logits, acts, questions, items):
                if items[0][3].get("fail") == "decode":
                    raise KeyError("decode")
                assert len(set(logits)) == 1  # this request's slice only
                return {q: logits[0] for q in questions}

            def close(self):
                script.threads.add(threading.get_ident())
                script.closed += 1

        monkeypatch.setattr(batching, "Engine", StandIn)
        return self


@pytest.fixture
def script(monkeypatch):
    return Script().install(monkeypatch)


def req(tag, *rows, fail=None):
    state = {"tag": tag, "rows": list(rows) or [20]}
    if fail:
        state["fail"] = fail
    return state, {f"q{i}": i for i in range(len(state["rows"]))}


def test_one_owner_thread_and_inputs_snapshotted(script):
    with BatchEngine(max_wait_ms=40) as engine:
        state, questions = req("a", 20, 30)
        first = engine.submit(state, questions)
        state["tag"] = "mutated"
        questions.clear()
        second = engine.submit(*req("b", 40))
        assert first.result(5) == {"q0": "a", "q1": "a"}
        assert second.result(5) == {"q0": "b"}
        m = first.metrics
        assert m["batch_requests"] == 2 and m["batch_questions"] == 3 and m["gpu_ms"] == 0.5
        assert m["tokens_per_question"] == [20, 30] and m["backend"] == "cuda"
        assert m["api_ms"] >= m["queue_ms"] >= 0
    assert script.packs == [["a", "b"]]
    assert len(script.threads) == 1 and threading.get_ident() not in script.threads
    assert script.closed == 1


def test_packs_follow_arrival_order_within_the_row_budget(script):
    # Rows are 16-aligned spans: 150 -> 160, 120 -> 128, 50 -> 64, 20 -> 32.  A 256-row budget
    # takes 160 + 64 + 32 in the first pack (the 128-row request does not fit after the first);
    # the skipped request runs next, alone.
    with BatchEngine(max_batch_tokens=256, max_wait_ms=50) as engine:
        futures = [engine.submit(*req(tag, n)) for tag, n in (("w", 150), ("x", 120), ("y", 50), ("z", 20))]
        assert [f.result(5) for f in futures] == [{"q0": t} for t in "wxyz"]
    assert script.packs == [["w", "y", "z"], ["x"]]
    assert [f.metrics["batch_requests"] for f in futures] == [3, 1, 3, 3]


def test_packs_follow_arrival_order_within_the_question_budget(script):
    with BatchEngine(max_batch_size=4, max_wait_ms=50) as engine:
        futures = [engine.submit(*req(tag, *([20] * q))) for tag, q in (("p", 3), ("q", 2), ("r", 1), ("s", 4))]
        for f in futures:
            f.result(5)
    assert script.packs == [["p", "r"], ["q"], ["s"]]


def test_each_failure_reaches_only_its_requests(script):
    with BatchEngine(max_batch_size=4, max_batch_tokens=512, max_wait_ms=0) as engine:
        with pytest.raises(ValueError, match="cannot prepare"):
            engine.submit(*req("bad", fail="prepare")).result(5)
        with pytest.raises(ValueError, match="cannot prepare"):
            engine.submit({"tag": "none", "rows": []}, {}).result(5)
        with pytest.raises(ValueError, match="batch budget"):
            engine.submit(*req("wide", *[20] * 5)).result(5)  # 5 questions > 4
        with pytest.raises(ValueError, match="batch budget"):
            engine.submit(*req("long", 600)).result(5)  # 608 rows > 512
        with pytest.raises(RuntimeError, match="device lost"):
            engine.submit(*req("lost", fail="predict")).result(5)
        with pytest.raises(KeyError):
            engine.submit(*req("garbled", fail="decode")).result(5)
        assert engine.submit(*req("fine")).result(5) == {"q0": "fine"}
    assert engine._outstanding == 0


def test_a_forward_failure_fails_its_whole_pack_only(script):
    script.gate.clear()
    engine = BatchEngine(max_wait_ms=0)
    blocker = engine.submit(*req("blocker"))
    assert script.busy.wait(5)
    doomed = [engine.submit(*req("lost", fail="predict")), engine.submit(*req("mate"))]
    script.gate.set()
    assert blocker.result(5) == {"q0": "blocker"}
    for f in doomed:
        with pytest.raises(RuntimeError, match="device lost"):
            f.result(5)
    assert engine.submit(*req("after")).result(5) == {"q0": "after"}
    engine.close()
    assert script.packs[1] == ["lost", "mate"]


def test_queue_bound_cancellation_and_close(script):
    script.gate.clear()
    engine = BatchEngine(max_pending=2, max_wait_ms=0)
    running = engine.submit(*req("running"))
    assert script.busy.wait(5)
    queued = engine.submit(*req("queued"))
    with pytest.raises(Full):
        engine.submit(*req("overflow"))
    assert queued.cancel()
    script.gate.set()
    engine.close()
    assert running.result() == {"q0": "running"} and queued.cancelled()
    assert script.packs == [["running"]]  # the cancelled request never reached the device
    assert engine._outstanding == 0
    engine.close()  # idempotent
    with pytest.raises(RuntimeError, match="closed"):
        engine.submit(*req("late"))


def test_close_drains_accepted_work(script):
    script.gate.clear()
    engine = BatchEngine(max_wait_ms=0)
    futures = [engine.submit(*req(f"t{i}")) for i in range(5)]
    closer = threading.Thread(target=engine.close)
    closer.start()
    script.gate.set()
    closer.join(10)
    assert not closer.is_alive()
    assert [f.result(0) for f in futures] == [{"q0": f"t{i}"} for i in range(5)]


def test_many_producers_and_close_from_a_callback(script):
    with BatchEngine(max_wait_ms=2) as engine:
        with ThreadPoolExecutor(8) as pool:
            futures = list(pool.map(lambda i: engine.submit(*req(f"n{i}")), range(96)))
        assert [f.result(5) for f in futures] == [{"q0": f"n{i}"} for i in range(96)]
        assert sorted(t for pack in script.packs for t in pack) == sorted(f"n{i}" for i in range(96))
        done = threading.Event()

        def on_done(_):
            engine.close()  # runs on the owner thread: must not join itself
            done.set()
        engine.submit(*req("last")).add_done_callback(on_done)
        assert done.wait(5)


def test_construction_failures(script, monkeypatch):
    def broken(*args, **kwargs):
        raise FileNotFoundError("no such checkpoint")
    monkeypatch.setattr(batching, "Engine", broken)
    with pytest.raises(FileNotFoundError, match="no such checkpoint"):
        BatchEngine()
    for bad in ({"max_batch_size": 0}, {"max_batch_tokens": 1.5}, {"max_pending": True}, {"max_wait_ms": -1},
                {"max_wait_ms": float("inf")}, {"backend": "official"}):
        with pytest.raises(ValueError):
            BatchEngine(**bad)


def test_fatal_error_on_the_owner_thread_reaches_every_waiter(script):
    script.gate.clear()
    engine = BatchEngine(max_wait_ms=0)
    fatal = engine.submit(*req("boom", fail="fatal"))
    assert script.busy.wait(5)
    cancelled = engine.submit(*req("cancelled"))
    waiting = engine.submit(*req("waiting"))
    assert cancelled.cancel()
    script.gate.set()
    done, not_done = wait([fatal, cancelled, waiting], timeout=5)
    assert not not_done
    for f in (fatal, waiting):
        with pytest.raises(SystemExit):
            f.result()
    with pytest.raises(RuntimeError, match="closed"):
        engine.submit(*req("after"))
    engine.close()
    assert engine._outstanding == 0 and script.closed == 1
