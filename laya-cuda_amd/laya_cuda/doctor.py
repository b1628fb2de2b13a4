"""`doctor`: is this machine ready to serve Laya models on the MI355X path?

The reference's doctor (laya_cuda/cli.py:118-176) checks CuPy, the CUDA driver, each GPU's compute
capability, NVRTC and cuBLAS, builds its kernels and optionally times a model.  The ROCm
counterpart checks what this runtime depends on instead:

  library   liblaya_hip.so loads and its ABI version matches this binding
  devices   every HIP device (name, architecture, HBM, CUs); gfx950 is the built architecture
  forward   a small seeded encoder runs through every kernel family on the chosen device: outputs
            finite, graph replay equal to the eager pass bit for bit, the no-allocation entry point
            equal to both, slot memory returned on close
  model     (optional) a checkpoint loads, its resident-weight footprint against free HBM, and the
            first and warm prediction times

Each check reports ok / warn / fail; the report passes when nothing failed.
"""
import ctypes as ct
import platform
import time

import numpy as np

from . import __version__, _lib

QUESTIONS = {"urgent": {"type": "noul", "instructions": "Does this need urgent attention?"}}


class Report:
    def __init__(self, echo=None):
        self.checks, self.echo = [], echo

    def add(self, name, status, detail):
        self.checks.append({"check": name, "status": status, "detail": detail})
        if self.echo:
            self.echo(f"  {status:<4}  {name}: {detail}")

    @property
    def passed(self):
        return all(c["status"] != "fail" for c in self.checks)


def _device_index(device):
    if device != "cuda" and not (device.startswith("cuda:") and device[5:].isdigit()):
        raise ValueError("device must be 'cuda' or 'cuda:N'")
    return int(device[5:]) if ":" in device else 0


def check_library(report):
    try:
        lib = _lib.load()
    except Exception as error:
        report.add("library", "fail", f"{type(error).__name__}: {error}")
        return None
    report.add("library", "ok", f"{_lib.LIBRARY.name} ABI {lib.laya_abi_version()}")
    return lib


def check_devices(report, lib, index):
    count = ct.c_int()
    if lib.laya_device_count(ct.byref(count)) != _lib.OK:
        report.add("devices", "fail", _lib.error())
        return False
    if count.value == 0:
        report.add("devices", "fail", "no HIP device found")
        return False
    chosen_ok = False
    for d in range(count.value):
        info = _lib.LayaDevice()
        if lib.laya_device_info(d, ct.byref(info)) != _lib.OK:
            report.add(f"device {d}", "fail", _lib.error())
            continue
        arch = info.arch.decode()
        detail = (f"{info.name.decode()}, {arch}, {info.compute_units} CUs, {info.hbm_bytes / 2**30:.1f} GiB HBM "
                  f"({info.free_bytes / 2**30:.1f} GiB free), {info.lds_bytes_per_cu // 1024} KiB LDS per CU")
        if info.supported:
            report.add(f"device {d}", "ok", detail)
        else:
            report.add(f"device {d}", "warn" if d != index else "fail",
                       f"{detail}; this library is built for gfx950 (MI355X)")
        chosen_ok |= d == index and bool(info.supported)
    if index >= count.value:
        report.add("devices", "fail", f"cuda:{index} does not exist ({count.value} device(s))")
    return chosen_ok


def check_forward(report, index):
    """A 2-layer d=256 encoder with two packed sequences and three questions: every kernel family
    (embedding+LN, MFMA GEMM epilogues, split-K, attention, add+LN, decision head) runs once."""
    from . import synthetic
    from .runtime import Runtime, pack, shape_class
    spec = synthetic.adapter(None, layers=2, width=256, heads=4, intermediate=1024, vocab=2000, positions=128,
                             max_len=128)
    rng = np.random.default_rng(1)
    sequences = [rng.integers(5, 2000, 100, dtype=np.int32), rng.integers(5, 2000, 37, dtype=np.int32)]
    questions = [(0, [3, 40, 99], 0), (1, [1, 5, 6, 36], 1), (0, [50, 51], 2)]
    started = time.perf_counter()
    rt = Runtime(spec, index, 2, weights=synthetic.weights(spec, seed=0))
    try:
        graph = rt.predict_sequences(sequences, questions)
        first_ms = (time.perf_counter() - started) * 1e3
        eager = rt.predict_sequences(sequences, questions, capture=False)
        key = shape_class(sequences, questions)
        m, b, k = key
        block = pack(sequences, questions, key, spec.pad, spec.vocab)
        logits = np.empty((b, k), np.float32)
        acts = np.empty((b, spec.n_act), np.float32)
        rc = _lib.load().laya_predict_static(
            rt._handle, block.ctypes.data_as(ct.POINTER(ct.c_int32)), ct.byref(_lib.LayaShape(m, b, k)),
            logits.ctypes.data_as(ct.POINTER(ct.c_float)), acts.ctypes.data_as(ct.POINTER(ct.c_float)), None)
        _lib.check(rc, rt._handle)
        n = len(questions)
        problems = []
        if not (np.isfinite(graph[0]).all() and np.isfinite(graph[1]).all()):
            problems.append("non-finite outputs")
        if not (np.array_equal(graph[0], eager[0]) and np.array_equal(graph[1], eager[1])):
            problems.append("graph replay differs from the eager pass")
        if not (np.array_equal(logits[:n], graph[0]) and np.array_equal(acts[:n], graph[1])):
            problems.append("the no-allocation entry point differs from predict")
        warm = min(rt.predict_sequences(sequences, questions)[2]["gpu_ms"] for _ in range(5))
    finally:
        rt.close()
    if rt.pool.used_bytes() != 0:
        problems.append("device memory still owned after close")
    if problems:
        report.add("forward", "fail", "; ".join(problems))
    else:
        report.add("forward", "ok", f"2-layer d=256 encoder, 3 questions: first {first_ms:.1f} ms (load, slot, graph "
                                    f"capture), warm {warm:.3f} ms on the device; replay == eager == static bit for bit")


def check_model(report, model, device):
    from .engine import Engine
    index = _device_index(device)
    started = time.perf_counter()
    with Engine(model, device=device) as engine:
        load = time.perf_counter() - started
        times = []
        for _ in range(3):
            s = time.perf_counter()
            engine.predict("Please refund my duplicate payment.", QUESTIONS)
            times.append((time.perf_counter() - s) * 1e3)
        owned = engine.last_metrics["owned_gpu_bytes"]
        info = _lib.LayaDevice()
        _lib.check(_lib.load().laya_device_info(index, ct.byref(info)))
    report.add(f"model {model}", "ok",
               f"load {load:.2f} s, {engine.adapter.layers} layers d={engine.adapter.width} "
               f"({engine.adapter.precision}), {owned / 2**20:.0f} MiB resident with one slot, "
               f"{info.free_bytes / 2**30:.1f} GiB HBM free; first {times[0]:.1f} ms, warm {min(times[1:]):.2f} ms")


def run(model=None, device="cuda:0", echo=None):
    """Run every check; returns the Report (``.passed``, ``.checks``)."""
    report = Report(echo)
    try:
        index = _device_index(device)
        lib = check_library(report)
        if lib is None:
            return report
        if not check_devices(report, lib, index):
            return report
        check_forward(report, index)
        if model is not None:
            check_model(report, model, device)
    except Exception as error:
        report.add("error", "fail", f"{type(error).__name__}: {error}")
    return report


def header():
    return f"laya-mi355x {__version__}, Python {platform.python_version()}, {platform.platform(terse=True)}"
