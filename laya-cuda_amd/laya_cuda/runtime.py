"""Runtime: resident weights and bounded shape slots, over liblaya_hip's C ABI.

Same interface as the reference's Runtime (laya_cuda/runtime.py:136-197):
``Runtime(adapter, device, max_cached_shapes)``, ``predict(items, capture=True) ->
(logits, acts, metrics)``, ``close()``, ``weights[name]``, ``pool.used_bytes()``,
``len(slots)``.  The device side - HBM arena, stream, one hipGraph per shape slot, LRU - is
owned by the native library; this module validates checkpoints and packs requests.

Packing follows Slot.fill (runtime.py:52-68): sequences back to back, each starting at a multiple
of 16 rows; ``positions`` run 0..span-1 inside a sequence; ``rows`` is -1 past the last one;
per question ``indices`` hold the absolute packed rows of its CLS token and option markers.
Beyond the reference, several questions may share one sequence (``predict_sequences``):
each question names its sequence, and its indices are offset by that sequence's start.
"""
import ctypes as ct

import numpy as np

from . import _lib


def span(tokens):
    """Rows start at multiples of 16 tokens, the attention tile."""
    return -(-tokens // 16) * 16


def _pow2(n, low):
    return max(low, 1 << (n - 1).bit_length())


def _round_rows(rows):
    step = 32 if rows <= 256 else 64 if rows <= 512 else 128
    return -(-rows // step) * step


def classes(items):
    """Shape class of reference-style items [(ids, markers, kind)]: one sequence per question."""
    rows = sum(span(len(v[0])) for v in items)
    return _round_rows(rows), _pow2(len(items), 1), _pow2(max(len(v[1]) for v in items), 8)


def shape_class(sequences, questions):
    """Shape class when questions share sequences: (rows, question capacity, option capacity)."""
    rows = sum(span(len(ids)) for ids in sequences)
    return (_round_rows(rows), _pow2(max(len(questions), len(sequences)), 1),
            _pow2(max(len(q[1]) for q in questions), 8))


def pack(sequences, questions, key, pad, vocab=None):
    """Packed int32 block for liblaya_hip (field order in include/laya_hip.h).

    Small requests are packed with a loop per sequence and per question (a few NumPy calls each);
    batches of more than PACK_LOOP_LIMIT sequences or questions with whole-array NumPy operations
    (per-question Python work dominated a 32-request batch: 760 -> 330 us on one host core).  Both
    forms write the same block and raise the same error for the first bad question."""
    m, b, k = key
    size = 4 + 4 * m + 4 * b + b * (k + 1)
    block = np.zeros(size, np.int32)
    o = 4
    ids, positions, rows, kinds = (block[o + i * m:o + (i + 1) * m] for i in range(4))
    o += 4 * m
    starts, lengths, counts, qkind = (block[o + i * b:o + (i + 1) * b] for i in range(4))
    indices = block[o + 4 * b:].reshape(b, k + 1)
    n_seq, n_q = len(sequences), len(questions)
    if n_seq > b or n_q > b:
        raise ValueError("More sequences or questions than the shape class holds")
    block[0], block[1] = n_seq, n_q
    ids.fill(pad)
    if max(n_seq, n_q) <= PACK_LOOP_LIMIT:
        _pack_loop(sequences, questions, m, k, ids, positions, rows, kinds, starts, lengths, counts, qkind, indices)
    else:
        _pack_arrays(sequences, questions, m, k, ids, positions, rows, kinds, starts, lengths, counts, qkind,
                     indices)
    if vocab is not None and n_seq and (ids.min() < 0 or ids.max() >= vocab):
        raise ValueError("Token id outside the vocabulary")
    return block


PACK_LOOP_LIMIT = 8


def _marker_error(q):
    return ValueError(f"Question {q} has option markers outside its sequence")


def _pack_loop(sequences, questions, m, k, ids, positions, rows, kinds, starts, lengths, counts, qkind, indices):
    rows.fill(-1)
    first_kind = {}
    for seq, _, kind in questions:
        first_kind.setdefault(seq, kind)
    offset = 0
    seq_start, seq_len = [], []
    for s, seq_ids in enumerate(sequences):
        n = len(seq_ids)
        end = offset + span(n)
        if end > m:
            raise ValueError("Packed sequences exceed the shape class")
        ids[offset:offset + n] = seq_ids
        positions[offset:end] = _RAMP[:end - offset] if end - offset <= _RAMP.size else np.arange(end - offset)
        rows[offset:end] = s
        kinds[offset:end] = first_kind.get(s, 0)
        seq_start.append(offset)
        seq_len.append(n)
        offset = end
    n_seq = len(sequences)
    starts[:n_seq], lengths[:n_seq] = seq_start, seq_len
    for q, (s, markers, kind) in enumerate(questions):
        if not 0 <= s < n_seq:
            raise ValueError(f"Question {q} names a missing sequence")
        cnt = len(markers)
        if cnt > k or (cnt and (min(markers) < 0 or max(markers) >= seq_len[s])):
            raise _marker_error(q)
        counts[q], qkind[q] = cnt, kind
        indices[q] = seq_start[s]
        indices[q, 1:cnt + 1] += np.asarray(markers, np.int32)


def _pack_arrays(sequences, questions, m, k, ids, positions, rows, kinds, starts, lengths, counts, qkind, indices):
    n_seq, n_q = len(sequences), len(questions)
    seq_len = np.fromiter(map(len, sequences), np.int64, n_seq)
    spans = (seq_len + 15) // 16 * 16
    seq_end = np.cumsum(spans)
    used = int(seq_end[-1]) if n_seq else 0
    if used > m:
        raise ValueError("Packed sequences exceed the shape class")
    seq_start = seq_end - spans
    starts[:n_seq], lengths[:n_seq] = seq_start, seq_len
    for s, seq_ids in enumerate(sequences):
        o = int(seq_start[s])
        ids[o:o + len(seq_ids)] = seq_ids
    rows[used:] = -1
    rows[:used] = np.repeat(np.arange(n_seq, dtype=np.int32), spans)
    positions[:used] = np.arange(used, dtype=np.int32) - np.repeat(seq_start.astype(np.int32), spans)
    seq_kind = np.zeros(n_seq, np.int64)
    if n_q:
        qseq = np.fromiter((q[0] for q in questions), np.int64, n_q)
        qk = np.fromiter((q[2] for q in questions), np.int64, n_q)
        if qk.min() < -2 ** 31 or qk.max() >= 2 ** 31:  # as the loop form's int32 stores refuse them
            raise OverflowError("Question kind out of int32 range")
        cnt = np.fromiter((len(q[1]) for q in questions), np.int64, n_q)
        total = int(cnt.sum())
        marks = np.fromiter((x for q in questions for x in q[1]), np.int64, total)
        # The first bad question in order, with the error the loop form raises for it.
        missing = (qseq < 0) | (qseq >= n_seq)
        bad = missing | (cnt > k)
        owner = np.repeat(np.arange(n_q), cnt)
        if total:
            limit = seq_len[np.where(missing, 0, qseq)][owner] if n_seq else np.zeros(total, np.int64)
            outside = (marks < 0) | (marks >= limit)
            bad[owner[outside]] = True
        if bad.any():
            q = int(np.flatnonzero(bad)[0])
            if missing[q]:
                raise ValueError(f"Question {q} names a missing sequence")
            raise _marker_error(q)
        counts[:n_q], qkind[:n_q] = cnt, qk
        indices[:n_q] = seq_start[qseq][:, None]
        if total:
            slot = np.arange(total) - np.repeat(np.cumsum(cnt) - cnt, cnt) + 1
            indices[owner, slot] += marks.astype(np.int32)
        # A sequence's token kinds are those of its first question (in question order).
        seqs_with, first_q = np.unique(qseq, return_index=True)
        seq_kind[seqs_with] = qk[first_q]
    kinds[:used] = np.repeat(seq_kind.astype(np.int32), spans)


_RAMP = np.arange(1 << 16, dtype=np.int32)


class _Resident:
    """Read-back handle for a resident tensor (mirrors a CuPy array's ``.get()``)."""

    def __init__(self, runtime, name, shape):
        self.runtime, self.name, self.shape = runtime, name, tuple(shape)

    def get(self):
        out = np.empty(self.shape, np.float32)
        ptr = out.ctypes.data_as(ct.POINTER(ct.c_float))
        _lib.check(_lib.load().laya_read_weight(self.runtime._handle, self.name.encode(), ptr, out.size),
                   self.runtime._handle)
        return out


class _Pool:
    def __init__(self, runtime):
        self.runtime = runtime

    def used_bytes(self):
        h = self.runtime._handle
        return int(_lib.load().laya_used_bytes(h)) if h else 0

    total_bytes = used_bytes


class _Slots:
    def __init__(self, runtime):
        self.runtime = runtime

    def __len__(self):
        h = self.runtime._handle
        return int(_lib.load().laya_slot_count(h)) if h else 0


def _config(adapter):
    precision = getattr(adapter, "mfma_dtype", "float16")
    bert = getattr(adapter, "variant", "modernbert") == "bert"
    return _lib.LayaConfig(
        width=adapter.width, heads=adapter.heads, layers=adapter.layers, intermediate=adapter.intermediate,
        vocab=adapter.vocab, max_positions=adapter.max_positions, type_vocab=adapter.type_vocab,
        norm_order=_lib.NORM_POST if bert else _lib.NORM_PRE,
        pos_kind=_lib.POS_LEARNED if bert else _lib.POS_ROPE,
        ffn_kind=_lib.FFN_GELU if bert else _lib.FFN_GEGLU, bias=int(bert), eps=adapter.eps,
        window=adapter.window if not bert else -1, global_every=adapter.global_every,
        head_layers=adapter.head_layers, n_act=adapter.n_act, act_hidden=adapter.act_hidden,
        max_len=adapter.max_len, mfma_dtype=_lib.F16 if precision == "float16" else _lib.BF16,
        theta_global=adapter.theta[0] if adapter.theta else 0.0,
        theta_local=adapter.theta[1] if len(adapter.theta) > 1 else 0.0)


def _host_dtype(array):
    if array.dtype == np.float32:
        return _lib.F32
    if array.dtype == np.float16:
        return _lib.F16
    raise ValueError(f"Unsupported checkpoint dtype {array.dtype}")


class Runtime:
    """One engine on one HIP device: weights resident in HBM, shape slots with hipGraphs."""

    def __init__(self, adapter, device, max_cached_shapes=16, *, weights=None):
        self.adapter, self.device, self.limit = adapter, device, max_cached_shapes
        self._handle = None
        self.pool, self.slots = _Pool(self), _Slots(self)
        self.weights = {}
        lib = _lib.load()
        handle = ct.c_void_p()
        config = _config(adapter)
        _lib.check(lib.laya_create(ct.byref(config), int(device), int(max_cached_shapes), ct.byref(handle)))
        self._handle = handle
        try:
            shapes = adapter.weight_shapes()
            if weights is None:
                from safetensors import safe_open
                with safe_open(str(adapter.path / "model.safetensors"), framework="numpy") as f:
                    self._load(shapes, set(f.keys()), lambda n: tuple(f.get_slice(n).get_shape()), f.get_tensor)
            else:
                self._load(shapes, set(weights), lambda n: tuple(np.shape(weights[n])), lambda n: weights[n])
            _lib.check(lib.laya_finalize(self._handle), self._handle)
        except BaseException:
            self.close()
            raise

    def _load(self, shapes, names, shape_of, tensor):
        if names != set(shapes):
            raise ValueError("Checkpoint tensor names do not match the Laya adapter")
        for name, shape in shapes.items():
            if shape_of(name) != tuple(shape):
                raise ValueError(f"Incompatible tensor shape: {name}")
        lib = _lib.load()
        for name, shape in shapes.items():
            if name == "temperature":
                continue
            array = np.ascontiguousarray(tensor(name))
            if array.dtype not in (np.float32, np.float16):
                array = array.astype(np.float32)
            dims = (ct.c_int64 * len(shape))(*shape)
            _lib.check(lib.laya_load_weight(self._handle, name.encode(), array.ctypes.data_as(ct.c_void_p),
                                            _host_dtype(array), dims, len(shape)), self._handle)
            self.weights[name] = _Resident(self, name, shape)

    def predict(self, items, capture=True):
        """Reference-style items [(ids, markers, kind)]: each question is its own sequence."""
        sequences = [ids for ids, _, _ in items]
        questions = [(i, markers, kind) for i, (_, markers, kind) in enumerate(items)]
        return self.predict_sequences(sequences, questions, capture, key=classes(items))

    def predict_sequences(self, sequences, questions, capture=True, key=None):
        """Questions [(sequence index, markers, kind)] over shared sequences."""
        if self._handle is None:
            raise RuntimeError("Runtime is closed")
        if not questions:
            raise ValueError("Provide at least one question")
        if self.adapter.head_layers:
            # Head transformer layers add each token's question-type row to the whole sequence
            # (laya.py:218), so a sequence can carry questions of one type only.
            kinds = {}
            for seq, _, kind in questions:
                if kinds.setdefault(seq, kind) != kind:
                    raise ValueError("With head transformer layers, questions sharing a sequence must share its type")
        key = key or shape_class(sequences, questions)
        block = pack(sequences, questions, key, self.adapter.pad, self.adapter.vocab)
        m, b, k = key
        logits = np.empty((b, k), np.float32)
        acts = np.empty((b, self.adapter.n_act), np.float32)
        shape = _lib.LayaShape(m, b, k)
        metrics = _lib.LayaMetrics()
        _lib.check(_lib.load().laya_predict(
            self._handle, block.ctypes.data_as(ct.POINTER(ct.c_int32)), ct.byref(shape), int(bool(capture)),
            logits.ctypes.data_as(ct.POINTER(ct.c_float)), acts.ctypes.data_as(ct.POINTER(ct.c_float)),
            ct.byref(metrics)), self._handle)
        n = len(questions)
        return logits[:n], acts[:n], {
            "gpu_ms": float(metrics.gpu_ms), "shape": key, "cache_miss": bool(metrics.cache_miss),
            "graph_capture": bool(metrics.graph_capture), "graph_replay": bool(metrics.graph_replay),
            "owned_gpu_bytes": int(metrics.owned_gpu_bytes)}

    @staticmethod
    def stages():
        """Names of the forward's launches, in order (per-layer stages run once per layer)."""
        lib = _lib.load()
        return [lib.laya_stage_name(i).decode() for i in range(lib.laya_stage_count())]

    def stage_launches(self, stage):
        """(launches per forward, first layer) of ``stage`` in this model; (0, -1) if it has none."""
        if self._handle is None:
            raise RuntimeError("Runtime is closed")
        index = self.stages().index(stage) if isinstance(stage, str) else int(stage)
        n, first = ct.c_int32(), ct.c_int32()
        _lib.check(_lib.load().laya_stage_launches(self._handle, index, ct.byref(n), ct.byref(first)), self._handle)
        return int(n.value), int(first.value)

    def time_stage(self, sequences, questions, stage, layer=0, reps=50, key=None):
        """Average device time (ms) of one launch of ``stage`` on this request's shape slot,
        measured with events around ``reps`` back-to-back launches on the engine's stream."""
        if self._handle is None:
            raise RuntimeError("Runtime is closed")
        key = key or shape_class(sequences, questions)
        block = pack(sequences, questions, key, self.adapter.pad, self.adapter.vocab)
        index = self.stages().index(stage) if isinstance(stage, str) else int(stage)
        avg = ct.c_float()
        _lib.check(_lib.load().laya_time_stage(
            self._handle, block.ctypes.data_as(ct.POINTER(ct.c_int32)), ct.byref(_lib.LayaShape(*key)), index,
            int(layer), int(reps), ct.byref(avg)), self._handle)
        return float(avg.value)

    def close(self):
        if self._handle is not None:
            _lib.load().laya_destroy(self._handle)
            self._handle = None
        self.weights = {}
