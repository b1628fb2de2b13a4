"""Shape classes and packing (laya_cuda/runtime.py:15-25, 52-67), checked by their closed forms
and invariants on small inputs (no GPU)."""
import numpy as np
import pytest

from laya_cuda import runtime
from laya_cuda.runtime import classes, pack, shape_class, span


@pytest.fixture(autouse=True, params=["loop", "arrays"])
def pack_form(request, monkeypatch):
    """Every test runs against both forms of pack (per-item loops for small requests, whole-array
    NumPy for batches), forced by the size limit between them."""
    monkeypatch.setattr(runtime, "PACK_LOOP_LIMIT", 1 << 30 if request.param == "loop" else -1)
    return request.param


def test_span_and_classes_closed_forms():
    assert [span(n) for n in (0, 1, 15, 16, 17, 83, 512)] == [0, 16, 16, 16, 32, 96, 512]
    # rows rounded in 32/64/128 steps; questions to a power of two >= 1; options >= 8
    assert classes([([0] * 83, [1, 2, 3, 4], 0)]) == (96, 1, 8)
    assert classes([([0] * 20, [1], 0)] * 3) == (96, 4, 8)
    assert classes([([0] * 250, [1] * 9, 0)]) == (256, 1, 16)
    assert classes([([0] * 260, [1], 0)]) == (320, 1, 8)
    assert classes([([0] * 513, [1], 0)]) == (640, 1, 8)
    assert shape_class([[0] * 512], [(0, [1] * 4, 0), (0, [1] * 6, 0)]) == (512, 2, 8)
    assert shape_class([[0] * 40] * 3, [(0, [1], 0)]) == (160, 4, 8)


def brute_force_fill(items, key, pad):
    """Element-by-element restatement of Slot.fill for reference-style items."""
    m, b, k = key
    ids, positions, rows, kinds = [pad] * m, [0] * m, [-1] * m, [0] * m
    starts, lengths, counts, indices = [0] * b, [0] * b, [0] * b, [0] * (b * (k + 1))
    offset = 0
    for r, (tok, markers, kind) in enumerate(items):
        n = len(tok)
        for i in range(span(n)):
            if i < n:
                ids[offset + i] = tok[i]
            positions[offset + i], rows[offset + i], kinds[offset + i] = i, r, kind
        starts[r], lengths[r], counts[r] = offset, n, len(markers)
        for j in range(k + 1):
            indices[r * (k + 1) + j] = offset + (markers[j - 1] if 1 <= j <= len(markers) else 0)
        offset += span(n)
    return ids, positions, rows, kinds, starts, lengths, counts, indices


@pytest.mark.parametrize("seed", range(5))
def test_pack_matches_brute_force_fill(seed):
    rng = np.random.default_rng(seed)
    items = []
    for _ in range(int(rng.integers(1, 6))):
        n = int(rng.integers(2, 70))
        markers = sorted(rng.integers(1, n, int(rng.integers(1, 10))).tolist())
        items.append((rng.integers(5, 100, n).tolist(), markers, int(rng.integers(0, 3))))
    key = classes(items)
    m, b, k = key
    block = pack([i[0] for i in items], [(q, i[1], i[2]) for q, i in enumerate(items)], key, pad=1, vocab=100)
    want = brute_force_fill(items, key, pad=1)
    o = 4
    got = [block[o + i * m:o + (i + 1) * m] for i in range(4)]
    o += 4 * m
    got += [block[o:o + b], block[o + b:o + 2 * b], block[o + 2 * b:o + 3 * b]]
    qkind = block[o + 3 * b:o + 4 * b]
    got.append(block[o + 4 * b:])
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert block[0] == len(items) and block[1] == len(items)
    np.testing.assert_array_equal(qkind[:len(items)], [i[2] for i in items])


def test_shared_sequence_questions_offset_by_their_sequence():
    seqs = [list(range(5, 25)), list(range(5, 45))]
    questions = [(1, [3, 4], 0), (0, [1], 2), (1, [39], 1)]
    key = shape_class(seqs, questions)
    m, b, k = key
    block = pack(seqs, questions, key, pad=0)
    indices = block[4 + 4 * m + 4 * b:].reshape(b, k + 1)
    assert indices[0, :3].tolist() == [32, 35, 36]
    assert indices[1, :2].tolist() == [0, 1]
    assert indices[2, :2].tolist() == [32, 71]
    assert (indices[0, 3:] == 32).all()


def test_pack_rejects_bad_requests():
    with pytest.raises(ValueError, match="markers outside"):
        pack([[1, 2, 3]], [(0, [3], 0)], (32, 1, 8), pad=0)
    with pytest.raises(ValueError, match="missing sequence"):
        pack([[1, 2, 3]], [(1, [1], 0)], (32, 2, 8), pad=0)
    with pytest.raises(ValueError, match="vocabulary"):
        pack([[1, 200]], [(0, [1], 0)], (32, 1, 8), pad=0, vocab=100)


def loop_pack(sequences, questions, key, pad):
    """Item-by-item packing of shared-sequence requests (the contract of pack, restated with plain
    loops over tokens, rows and option slots)."""
    m, b, k = key
    ids, positions, rows, kinds = [pad] * m, [0] * m, [-1] * m, [0] * m
    starts, lengths, counts, qkind = [0] * b, [0] * b, [0] * b, [0] * b
    indices = [0] * (b * (k + 1))
    seq_kind = {}
    for s, _, kind in questions:
        if s not in seq_kind:
            seq_kind[s] = kind
    offset = 0
    for s, tok in enumerate(sequences):
        for i in range(span(len(tok))):
            if i < len(tok):
                ids[offset + i] = int(tok[i])
            positions[offset + i], rows[offset + i], kinds[offset + i] = i, s, seq_kind.get(s, 0)
        starts[s], lengths[s] = offset, len(tok)
        offset += span(len(tok))
    for q, (s, markers, kind) in enumerate(questions):
        counts[q], qkind[q] = len(markers), kind
        for j in range(k + 1):
            indices[q * (k + 1) + j] = starts[s] + (markers[j - 1] if 1 <= j <= len(markers) else 0)
    return [len(sequences), len(questions), 0, 0] + ids + positions + rows + kinds + starts + lengths + counts + qkind + indices


@pytest.mark.parametrize("seed", range(8))
def test_pack_of_shared_sequences_matches_a_loop_restatement(seed):
    """Several questions per sequence (duplicated and unsorted markers, differing kinds, sequences no
    question names, sequences of 1 and 16k tokens): the vectorised pack equals the loops."""
    rng = np.random.default_rng(100 + seed)
    sequences = [rng.integers(5, 1000, int(n)).tolist() for n in rng.choice([1, 15, 16, 17, 40, 333], 6)]
    questions = []
    for _ in range(int(rng.integers(1, 12))):
        s = int(rng.integers(0, len(sequences)))
        n = len(sequences[s])
        questions.append((s, rng.integers(0, n, int(rng.integers(0, 9))).tolist(), int(rng.integers(0, 3))))
    key = shape_class(sequences, questions) if any(q[1] for q in questions) else (1024, 16, 8)
    np.testing.assert_array_equal(pack(sequences, questions, key, pad=3), loop_pack(sequences, questions, key, pad=3))


def test_pack_reports_the_first_bad_question_in_order():
    seqs = [[5] * 10, [6] * 20]
    marker_first = [(0, [1], 0), (1, [25], 0), (7, [1], 0)]
    with pytest.raises(ValueError, match="Question 1 has option markers outside"):
        pack(seqs, marker_first, (64, 4, 8), pad=0)
    missing_first = [(0, [1], 0), (-1, [1], 0), (0, [-2], 0)]
    with pytest.raises(ValueError, match="Question 1 names a missing sequence"):
        pack(seqs, missing_first, (64, 4, 8), pad=0)
    with pytest.raises(ValueError, match="Question 0 has option markers outside"):
        pack(seqs, [(1, list(range(9)), 0)], (64, 4, 8), pad=0)  # more options than slots
    with pytest.raises(ValueError, match="exceed the shape class"):
        pack(seqs, [(0, [1], 0)], (16, 4, 8), pad=0)
    with pytest.raises(ValueError, match="missing sequence"):
        pack([], [(0, [1], 0)], (16, 1, 8), pad=0)


def test_a_sequence_takes_the_kind_of_its_first_question():
    seqs = [[5] * 10, [6] * 20, [7] * 3]
    questions = [(1, [2], 2), (0, [1], 1), (1, [3], 0)]
    m, b, k = key = (64, 4, 8)
    kinds = pack(seqs, questions, key, pad=0)[4 + 3 * m:4 + 4 * m]
    assert kinds[:16].tolist() == [1] * 16 and kinds[16:48].tolist() == [2] * 32
    assert kinds[48:64].tolist() == [0] * 16  # no question names the third sequence


def test_pack_refuses_kinds_outside_int32():
    with pytest.raises(OverflowError):
        pack([[5] * 10], [(0, [1], 2 ** 32 + 1)], (64, 4, 8), pad=0)
