"""Cross-request batching over one Engine (the reference's BatchEngine contract,
laya_cuda/batching.py:17-157).

Contract kept from the reference: ``BatchEngine(model, *, max_batch_size, max_batch_tokens,
max_pending, max_wait_ms, **engine_options)``, ``submit(state, questions) -> Future`` whose
``.metrics`` carries the runtime metrics plus ``batch_questions``, ``batch_requests``,
``queue_ms``, ``api_ms``, ``tokens_per_question``, ``backend`` and ``precision``; ``close()``
refuses new work and drains accepted work; a full queue raises ``queue.Full``; a closed engine
raises ``RuntimeError``; the device has one owner thread; requests pack in arrival order within
the question and packed-row budgets; a failure reaches only the requests it concerns.

Design: a ``_Ticket`` per request travels through three phases on the owner thread -
``_next_window`` (block for the first ticket, then linger until the oldest ticket's deadline or a
full window), ``_admit`` (cancellation check, ``prepare``, budget check) and ``_run`` (one
``Runtime.predict`` per pack, then per-ticket decode).  Every ticket is settled exactly once
(``_settle``); a fatal error on the owner thread settles whatever is still unsettled with that
error and closes the engine for new work.
"""
from collections import deque
from concurrent.futures import Future
from copy import deepcopy
from dataclasses import dataclass, field
import math
from queue import Full
import threading
import time

from .engine import Engine


class _Prediction(Future):
    """A Future with the per-request ``metrics`` dict of the reference's BatchEngine."""
    metrics: dict


@dataclass(eq=False)
class _Ticket:
    future: _Prediction
    state: object
    questions: object
    submitted: float
    items: list = field(default_factory=list)  # prepared (ids, markers, kind) rows
    rows: int = 0                               # packed rows these items occupy
    settled: bool = False


def _packs(tickets, max_questions, max_rows):
    """Split admitted tickets into packs: each pack takes, in arrival order, every remaining ticket
    that still fits its question and row budgets; the skipped ones form the following packs.
    Every ticket fits an empty pack (``_admit`` checked that), so no pack is empty."""
    remaining = list(tickets)
    while remaining:
        pack, later, questions, rows = [], [], 0, 0
        for ticket in remaining:
            fits = questions + len(ticket.items) <= max_questions and rows + ticket.rows <= max_rows
            if fits:
                pack.append(ticket)
                questions += len(ticket.items)
                rows += ticket.rows
            else:
                later.append(ticket)
        yield pack
        remaining = later


class BatchEngine:
    def __init__(self, model="laya", *, max_batch_size=16, max_batch_tokens=4096, max_pending=128, max_wait_ms=1,
                 **engine_options):
        limits = (max_batch_size, max_batch_tokens, max_pending)
        if any(type(v) is not int or v < 1 for v in limits):
            raise ValueError("Batch and queue limits must be positive integers")
        if not (isinstance(max_wait_ms, (int, float)) and math.isfinite(max_wait_ms) and max_wait_ms >= 0):
            raise ValueError("max_wait_ms must be finite and nonnegative")
        if engine_options.get("backend", "cuda") != "cuda":
            raise ValueError("BatchEngine supports backend='cuda' only")
        self.max_batch_size, self.max_batch_tokens, self.max_pending = limits
        self.linger = max_wait_ms / 1000.0
        self._lock = threading.Lock()
        self._wake = threading.Condition(self._lock)
        self._inbox = deque()
        self._outstanding = 0  # accepted and not yet settled
        self._closing = False
        booted = Future()
        self._owner = threading.Thread(target=self._serve, args=(model, engine_options, booted),
                                       name="laya-batch", daemon=True)
        self._owner.start()
        booted.result()  # re-raises an Engine construction failure here

    # ---- caller side -------------------------------------------------------------------------
    def submit(self, state, questions):
        """Queue a request; returns a Future (with ``.metrics``).  Raises queue.Full at the
        pending limit and RuntimeError once closed.  The inputs are copied at submission."""
        now = time.perf_counter()
        with self._lock:
            if self._closing:
                raise RuntimeError("BatchEngine is closed")
            if self._outstanding >= self.max_pending:
                raise Full("BatchEngine pending request limit reached")
            future = _Prediction()
            future.metrics = {}
            self._inbox.append(_Ticket(future, deepcopy(state), deepcopy(questions), now))
            self._outstanding += 1
            self._wake.notify()
        return future

    def close(self):
        """Stop accepting requests, finish every accepted one, release the device."""
        with self._lock:
            self._closing = True
            self._wake.notify_all()
        if threading.current_thread() is not self._owner:
            self._owner.join()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- owner thread ------------------------------------------------------------------------
    def _settle(self, ticket, result=None, error=None):
        with self._lock:
            if ticket.settled:
                return
            ticket.settled = True
            self._outstanding -= 1
        future = ticket.future
        if future.cancelled():
            return
        if error is not None:
            future.set_exception(error)
        else:
            future.set_result(result)

    def _next_window(self):
        """The tickets of the next batching window, or None once closed with nothing queued."""
        with self._lock:
            while not self._inbox and not self._closing:
                self._wake.wait()
            if not self._inbox:
                return None
            deadline = self._inbox[0].submitted + self.linger
            while not self._closing and len(self._inbox) < self.max_batch_size:
                left = deadline - time.perf_counter()
                if left <= 0 or not self._wake.wait(left):
                    break
            window = list(self._inbox)
            self._inbox.clear()
            return window

    def _admit(self, engine, ticket, span):
        """Claim, prepare and budget-check one ticket; False (ticket settled) if it drops out."""
        if not ticket.future.set_running_or_notify_cancel():
            self._settle(ticket)  # cancelled while queued
            return False
        try:
            ticket.items = engine.adapter.prepare(ticket.state, ticket.questions)
            ticket.rows = sum(span(len(item[0])) for item in ticket.items)
            if len(ticket.items) > self.max_batch_size or ticket.rows > self.max_batch_tokens:
                raise ValueError("Request exceeds batch budget; increase limits or submit fewer questions")
        except Exception as error:
            self._settle(ticket, error=error)
            return False
        return True

    def _run(self, engine, pack):
        """One forward for the pack, then each ticket's slice of logits and acts is decoded."""
        items = [item for ticket in pack for item in ticket.items]
        launched = time.perf_counter()
        try:
            logits, acts, metrics = engine.runtime.predict(items)
        except Exception as error:
            for ticket in pack:
                self._settle(ticket, error=error)
            return
        precision = getattr(engine.adapter, "precision", "float16")
        first = 0
        for ticket in pack:
            rows = slice(first, first + len(ticket.items))
            first = rows.stop
            try:
                answer = engine.adapter.decode(logits[rows], acts[rows], ticket.questions, ticket.items)
            except Exception as error:
                self._settle(ticket, error=error)
                continue
            ticket.future.metrics = {
                **metrics, "batch_questions": len(items), "batch_requests": len(pack),
                "queue_ms": (launched - ticket.submitted) * 1e3, "api_ms": (time.perf_counter() - ticket.submitted) * 1e3,
                "tokens_per_question": [len(item[0]) for item in ticket.items], "backend": "cuda",
                "precision": precision}
            self._settle(ticket, answer)

    def _serve(self, model, options, booted):
        engine, window = None, []
        try:
            engine = Engine(model, **options)
            from .runtime import span  # the native library is loaded by now
            booted.set_result(None)
            while True:
                window = self._next_window()
                if window is None:
                    break
                admitted = [t for t in window if self._admit(engine, t, span)]
                for pack in _packs(admitted, self.max_batch_size, self.max_batch_tokens):
                    self._run(engine, pack)
                window = []
        except BaseException as error:  # also KeyboardInterrupt/SystemExit raised inside a forward
            with self._lock:
                self._closing = True
                stranded = window + list(self._inbox)
                self._inbox.clear()
            if not booted.done():
                booted.set_exception(error)
            for ticket in stranded:
                if ticket.settled:
                    continue
                if not ticket.future.running():
                    ticket.future.set_running_or_notify_cancel()  # wakes wait() on cancelled futures
                self._settle(ticket, error=error)
        finally:
            if engine is not None:
                engine.close()
