"""Laya.prepare: tokenisation, option markers and context budget (laya_cuda/laya.py:104-135 of the
reference), on a checkpoint directory whose tokenizer is trained here (no real tokenizer.json is
available offline, so byte-level parity with a Laya tokenizer stays unpinned; what is checked is
the token layout the encoder and decision head rely on).

Layout of one question: [CLS] head [SEP] ([MASK] option-tokens)* [SEP] state-tokens [SEP], cut to
max_len; head = "<type> question: <instructions>", each option at most 48 tokens after its
[MASK], the head at least 8 tokens and otherwise what head_max_len leaves after the options."""
import pytest

from synthetic_checkpoint import write

from laya_cuda.laya import Laya, question


@pytest.fixture(scope="module")
def laya(tmp_path_factory):
    path, _, _ = write(tmp_path_factory.mktemp("checkpoint"), max_len=128, head_max_len=48)
    return Laya(path)


def enc(laya, text):
    return laya.tokenizer.encode(text, add_special_tokens=False).ids


def segments(laya, ids, markers):
    """(head, [option segments], state) of one prepared question."""
    assert ids[0] == laya.cls and ids[markers[0] - 1] == laya.sep
    end = ids.index(laya.sep, markers[-1])  # first [SEP] after the last option
    bounds = markers + [end]
    return ids[1:markers[0] - 1], [ids[a:b] for a, b in zip(bounds, bounds[1:])], ids[end + 1:]


QUESTIONS = {
    "route": {"type": "choice", "instructions": "Choose a team for the ticket",
              "criteria": {"billing": "invoices and payment errors", "shipping": "delivery and tracking", "other": None}},
    "angry": {"type": "noul", "instructions": "Is the customer angry?"},
    "urgency": {"type": "score", "instructions": "How urgent is the ticket?",
                "criteria": ["not urgent", "urgent", "critical"]},
}


def test_token_contract(laya):
    """tests/test_contract.py:97-108 of the reference, on this checkpoint."""
    queries = {"q": {"type": "choice", "instructions": "Choose [MASK] a team", "criteria": {"billing": "payment", "other": None}}}
    seq, markers, kind = laya.prepare("refund " * 5000, queries)[0]
    assert len(seq) == laya.max_len and seq[0] == laya.cls and seq[-1] == laya.sep
    assert len(markers) == 2 and all(seq[i] == laya.mask for i in markers) and kind == 0
    with pytest.raises(ValueError):
        laya.prepare("", {})


def test_segments_are_the_texts_own_tokens(laya):
    state = "the customer asks about a late delivery and wants a refund"
    items = laya.prepare(state, QUESTIONS)
    assert [kind for _, _, kind in items] == [0, 2, 1]  # TYPES order: choice, score, noul
    for (ids, markers, _), definition in zip(items, QUESTIONS.values()):
        kind, instruction, _, options = question(definition)
        head, opts, tail = segments(laya, ids, markers)
        assert len(opts) == len(options)
        for seg, option in zip(opts, options):
            assert seg[0] == laya.mask and 1 <= len(seg) <= 49
            assert seg[1:] == enc(laya, " " + option)[:len(seg) - 1]
        want_head = enc(laya, f"{kind} question: {instruction}")
        assert head == want_head[:max(8, laya.head_max_len - sum(map(len, opts)))]
        assert tail == enc(laya, state) + [laya.sep]  # short state: all of it, then [SEP]
        assert len(ids) <= laya.max_len


def test_long_options_are_capped_to_the_head_budget(laya):
    """Options that leave fewer than 16 head tokens are cut to max(4, (head_max_len - 16) // n)."""
    long_text = "billing team handles invoices and payment errors " * 12
    q = {"q": {"type": "choice", "instructions": "route the ticket", "criteria": {f"team{i}": long_text for i in range(8)}}}
    ids, markers, _ = laya.prepare("refund", q)[0]
    _, opts, _ = segments(laya, ids, markers)
    cap = max(4, (laya.head_max_len - 16) // 8)
    assert all(len(seg) == cap for seg in opts)
    head_budget = max(8, laya.head_max_len - cap * 8)
    assert markers[0] - 2 == min(len(enc(laya, "choice question: route the ticket")), head_budget)


def test_mask_text_in_inputs_cannot_forge_markers(laya):
    state = "refund [MASK] the payment [MASK]"
    q = {"q": {"type": "choice", "instructions": "pick [MASK] one", "criteria": {"a [MASK]": "b [MASK]", "c": None}}}
    ids, markers, _ = laya.prepare(state, q)[0]
    assert [i for i, t in enumerate(ids) if t == laya.mask] == markers


def test_batched_encoding_matches_single_question_encoding(laya):
    """Twelve or more texts take the tokenizer's batch path; each text still encodes alone."""
    many = {f"q{i}": dict(QUESTIONS["route"], instructions=f"Choose a team for ticket {i}") for i in range(4)}
    state = {"ticket": "late delivery", "order": 1234, "notes": ["refund", "billing"]}  # JSON state
    batched = laya.prepare(state, many)
    for (qid, definition), item in zip(many.items(), batched):
        assert laya.prepare(state, {qid: definition})[0] == item


def test_option_budget_overflow_raises(laya, monkeypatch):
    monkeypatch.setattr(laya, "max_len", 20)
    long_text = "shipping team handles delivery and tracking " * 4
    q = {"q": {"type": "choice", "instructions": "route", "criteria": {"a": long_text, "b": long_text}}}
    with pytest.raises(ValueError, match="exceeds the option token budget"):
        laya.prepare("refund", q)


def test_options_keep_at_most_48_tokens(laya, monkeypatch):
    """With room in the head budget, a long option keeps exactly its first 48 tokens."""
    monkeypatch.setattr(laya, "head_max_len", 120)
    long_text = "shipping team handles delivery and tracking " * 10
    q = {"q": {"type": "choice", "instructions": "route the ticket", "criteria": {"long": long_text, "short": None}}}
    ids, markers, _ = laya.prepare("refund", q)[0]
    _, (first, second), _ = segments(laya, ids, markers)
    assert len(enc(laya, " long: " + long_text)) > 48
    assert first == [laya.mask] + enc(laya, " long: " + long_text)[:48]
    assert second == [laya.mask] + enc(laya, " short")
    assert markers[0] - 2 == len(enc(laya, "choice question: route the ticket"))  # 120 - 51 tokens leave room


# ---- the state encoded from a prefix: the same first max_len ids as the whole text -------------

def _trained(pre_tokenizer, normalizer=None, model="bpe"):
    """A tokenizer trained here on the checkpoint corpus with the given pipeline stages."""
    from tokenizers import Tokenizer, models, trainers
    from laya_cuda import synthetic
    if model == "wordpiece":
        tok = Tokenizer(models.WordPiece(unk_token="[UNK]"))
        trainer = trainers.WordPieceTrainer(vocab_size=400, special_tokens=synthetic.TOKENIZER_SPECIALS)
    else:
        tok = Tokenizer(models.BPE(unk_token="[UNK]"))
        trainer = trainers.BpeTrainer(vocab_size=400, special_tokens=synthetic.TOKENIZER_SPECIALS)
    if normalizer is not None:
        tok.normalizer = normalizer
    if pre_tokenizer is not None:
        tok.pre_tokenizer = pre_tokenizer
    tok.train_from_iterator(synthetic.TOKENIZER_CORPUS * 10, trainer)
    return tok


def _pipelines():
    from tokenizers import normalizers, pre_tokenizers
    return {
        "whitespace": _trained(pre_tokenizers.Whitespace()),
        "byte-level": _trained(pre_tokenizers.ByteLevel(add_prefix_space=False)),
        "metaspace": _trained(pre_tokenizers.Metaspace()),
        "bert": _trained(pre_tokenizers.BertPreTokenizer(), normalizers.BertNormalizer(lowercase=True),
                         model="wordpiece"),
        "nfkc-sequence": _trained(pre_tokenizers.Sequence([pre_tokenizers.WhitespaceSplit(),
                                                           pre_tokenizers.Digits(individual_digits=True)]),
                                  normalizers.Sequence([normalizers.NFKC(), normalizers.Lowercase()])),
    }


def _random_text(rng, words):
    pieces = ["refund", "the", "customer", "payment", "délivery", "naïve", "ﬁle", "ÉCOLE", "12345", "3.5%",
              "don't", "e-mail", "软件错误", "😀", "ünïcödé", "[MASK]", "(note)", "—", "a", "x" * 40]
    seps = [" ", " ", " ", "  ", "\t", "\n", " \n ", ", ", ". ", "", "   "]
    return "".join(pieces[rng.integers(len(pieces))] + seps[rng.integers(len(seps))] for _ in range(words))


def test_state_prefix_encodes_to_the_whole_texts_leading_ids():
    """For every pipeline whose pre-tokenizer splits in front of a space after a letter or digit,
    the state ids prepare uses (the first max_len) are those of the whole text, on random texts of
    mixed scripts, digits, punctuation, runs of whitespace and an added-token string."""
    import json
    import numpy as np
    from laya_cuda.laya import _splits_at_spaces

    class Spec:
        pass

    rng = np.random.default_rng(7)
    for name, tok in _pipelines().items():
        assert _splits_at_spaces(json.loads(tok.to_str())), name
        for max_len in (16, 128, 512, 1024):
            spec = Spec()
            spec.tokenizer, spec.max_len, spec.prefix_cut = tok, max_len, True
            for words in (3, 200, 3000):
                text = _random_text(rng, words)
                whole = tok.encode(text, add_special_tokens=False).ids
                ids = Laya.state_ids(spec, text)
                # every id of the prefix's encoding, up to the cut, is the whole text's
                assert len(ids) >= min(max_len, len(whole)) and ids == whole[:len(ids)], (name, max_len, words)


def test_state_prefix_cut_is_off_for_tokenizers_that_join_across_spaces():
    """No pre-tokenizer (the whole text is one piece), a normaliser that rewrites patterns, or an
    added token containing a space: the whole text is encoded."""
    import json
    from tokenizers import AddedToken, normalizers, pre_tokenizers
    from laya_cuda.laya import _splits_at_spaces
    assert not _splits_at_spaces(json.loads(_trained(None).to_str()))
    assert not _splits_at_spaces(json.loads(_trained(pre_tokenizers.Whitespace(),
                                                     normalizers.Replace(" ", "_")).to_str()))
    assert not _splits_at_spaces(json.loads(_trained(pre_tokenizers.Punctuation()).to_str()))
    tok = _trained(pre_tokenizers.Whitespace())
    tok.add_tokens([AddedToken("late delivery")])
    assert not _splits_at_spaces(json.loads(tok.to_str()))
    # pieces after the first start with a space: a normaliser that strips it, or an added token
    # that swallows the space after it, would encode that space differently from the whole text
    assert not _splits_at_spaces(json.loads(_trained(pre_tokenizers.ByteLevel(), normalizers.Strip()).to_str()))
    tok = _trained(pre_tokenizers.ByteLevel())
    tok.add_tokens([AddedToken("refund9", rstrip=True)])
    assert not _splits_at_spaces(json.loads(tok.to_str()))


def test_prepare_is_unchanged_by_the_prefix_cut(laya):
    """prepare with the prefix cut equals prepare encoding the whole state, for long states."""
    import numpy as np
    rng = np.random.default_rng(9)
    assert laya.prefix_cut
    for words in (10, 400, 5000):
        state = _random_text(rng, words)
        fast = laya.prepare(state, QUESTIONS)
        laya.prefix_cut = False
        try:
            slow = laya.prepare(state, QUESTIONS)
        finally:
            laya.prefix_cut = True
        assert fast == slow


def test_a_cut_inside_a_word_breaks_the_prefix_property():
    """The check above can fail: cutting "refund" after "ref" encodes a different last token."""
    tok = _pipelines()["byte-level"]
    text = "refund " * 200
    whole = tok.encode(text, add_special_tokens=False).ids
    bad = tok.encode(text[:7 * 100 + 3], add_special_tokens=False).ids
    good = tok.encode(text[:7 * 100 + 6], add_special_tokens=False).ids
    assert bad != whole[:len(bad)] and good == whole[:len(good)]


def test_state_pieces_join_to_the_whole_texts_ids():
    """Texts whose first piece yields fewer than max_len ids are encoded in several pieces (each
    after the first starting with the space it was cut at); the joined ids are the whole text's."""
    import numpy as np

    class Counting:
        def __init__(self, tok):
            self.tok, self.calls = tok, 0

        def encode(self, text, add_special_tokens=False):
            self.calls += 1
            return self.tok.encode(text, add_special_tokens=add_special_tokens)

    class Spec:
        pass

    rng = np.random.default_rng(11)
    for name, tok in _pipelines().items():
        for text in ("refund " * 3000, "refund  payment\t" * 1500, " ".join(["x" * 40] * 400) + " end",
                     _random_text(rng, 4000).replace("软件错误", "refund")):
            for max_len in (512, 1024):
                spec = Spec()
                spec.tokenizer, spec.max_len, spec.prefix_cut = Counting(tok), max_len, True
                whole = tok.encode(text, add_special_tokens=False).ids
                ids = Laya.state_ids(spec, text)
                assert len(ids) >= min(max_len, len(whole)) and ids == whole[:len(ids)], (name, max_len)
        spec = Spec()
        spec.tokenizer, spec.max_len, spec.prefix_cut = Counting(tok), 1024, True
        Laya.state_ids(spec, "refund " * 3000)
        assert spec.tokenizer.calls >= 2, name  # the several-piece path ran
