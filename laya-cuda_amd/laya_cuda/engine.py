"""Public synchronous inference API (laya_cuda/engine.py:7-51 of the reference)."""
import time

from .models import adapter, resolve


class Engine:
    def __init__(self, model="laya", *, revision=None, device="cuda:0", backend="cuda", max_cached_shapes=16,
                 registry=None):
        if backend != "cuda":
            raise ValueError("backend must be 'cuda' (the HIP runtime); the official SDK backend is not available")
        if type(max_cached_shapes) is not int or not 1 <= max_cached_shapes <= 64:
            raise ValueError("max_cached_shapes must be an integer between 1 and 64")
        if device != "cuda" and not (device.startswith("cuda:") and device[5:].isdigit()):
            raise ValueError("v1 requires a GPU device 'cuda' or 'cuda:N' (HIP devices keep torch's naming)")
        self.backend, self.device, self.closed = backend, device, False
        self.last_metrics = {}
        self.path = resolve(model, revision, registry=registry)
        self.adapter = adapter(self.path)
        from .runtime import Runtime
        index = int(device.split(":")[-1]) if ":" in device else 0
        self.runtime = Runtime(self.adapter, index, max_cached_shapes)

    def predict(self, state, questions):
        if self.closed:
            raise RuntimeError("Engine is closed")
        started = time.perf_counter()
        items = self.adapter.prepare(state, questions)
        logits, acts, metrics = self.runtime.predict(items)
        result = self.adapter.decode(logits, acts, questions, items)
        metrics.update(precision=self.adapter.precision, tokens_per_question=[len(v[0]) for v in items],
                       input_sha256=self.adapter.fingerprint(items))
        self.last_metrics = {**metrics, "backend": self.backend, "api_ms": (time.perf_counter() - started) * 1000}
        return result

    def close(self):
        if not self.closed:
            self.runtime.close()
            self.closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
