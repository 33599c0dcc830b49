"""The C++ decision front end (libgliner_decide_frontend.so) on the CPU.

Pins:
* the tokenizer.json pipeline against the HF `tokenizers` library, id for id,
  on a sentencepiece Unigram model trained here with the nmt_nfkc rule (its
  precompiled charsmap is the genuine one) and assembled the way
  transformers' DebertaV2Converter assembles the checkpoint's tokenizer.json
  (Strip, Precompiled, Replace " {2,}", Metaspace), on fuzzed text over the
  vocabulary and over characters the normaliser rewrites (ligatures,
  full-width forms, combining marks, CR LF, controls, emoji sequences);
* the other normaliser / pre-tokenizer forms and the WordLevel model the
  same way;
* the Viterbi on a hand-scored vocabulary (best split, ties, fused unknowns);
* the word split (ICU, the engine behind NSRegularExpression) against the
  Python `regex` restatement of the same pattern, and the decision input
  (ids, mask, markers) against the HF-backed front end;
* the error cases of NativeTokenizerError and of the C-ABI.
"""

import ctypes as C
import json
import re
from pathlib import Path

import numpy as np
import pytest

from gliner_decide import _frontend_native as F
from gliner_decide.decode import DecisionTask
from gliner_decide.frontend import NativeDecisionTokenizer, TokenizerError, split_words

HEADER = Path(__file__).resolve().parents[1] / "include" / "gliner_decide_frontend.h"
SPECIALS = ["[PAD]", "[CLS]", "[SEP]", "[UNK]", "[MASK]"]
MARKERS = ["[P]", "[L]", "[SEP_STRUCT]", "[SEP_TEXT]", "[DESCRIPTION]"]
EXOTIC = list("éüñçÅØßΣσςİıĲ") + ["́", "̈", "‍", "​", "\t", "\n", "\r", "　", " ",
                                   "ﬁ", "①", "Ａ", "ｶ", "㍻", "東", "京", "\U0001f44d",
                                   "\U0001f3fd", "▁", "\x01", "\x7f", "﻿", "�", "한", "ᄀ",
                                   "ᅡ", "क", "्", "ष", "～", "~", "؀", "ﷺ"]


def _corpus(seed, count=20000):
    import random
    r = random.Random(seed)
    syl = ["ka", "re", "mo", "tion", "ing", "pre", "con", "ab", "st", "ly", "er", "ou", "ch", "sh", "qu", "x",
           "zz", "é", "ü", "ß", "ø", "ñ", "ç", "東", "京", "語", "한", "국", "д", "ж", "ы", "α", "β", "ω"]
    words = ["".join(r.choice(syl) for _ in range(r.randint(1, 4))) for _ in range(3000)]
    lines = []
    for _ in range(count):
        ws = [r.choice(words) for _ in range(r.randint(3, 20))]
        ws = [w.capitalize() if r.random() < 0.2 else w for w in ws]
        lines.append(" ".join(ws) + r.choice([".", "!", "?", ",", ""]))
    return lines


@pytest.fixture(scope="session")
def spm_parts(tmp_path_factory):
    spm = pytest.importorskip("sentencepiece")
    from sentencepiece import sentencepiece_model_pb2 as pb
    d = tmp_path_factory.mktemp("spm")
    (d / "corpus.txt").write_text("\n".join(_corpus(1)), encoding="utf-8")
    spm.SentencePieceTrainer.train(input=str(d / "corpus.txt"), model_prefix=str(d / "m"), vocab_size=2000,
                                   hard_vocab_limit=False, model_type="unigram", character_coverage=0.9995,
                                   normalization_rule_name="nmt_nfkc", pad_id=0, bos_id=1, eos_id=2, unk_id=3,
                                   pad_piece="[PAD]", bos_piece="[CLS]", eos_piece="[SEP]", unk_piece="[UNK]",
                                   minloglevel=2)
    m = pb.ModelProto()
    m.ParseFromString((d / "m.model").read_bytes())
    return [(p.piece, p.score) for p in m.pieces], m.normalizer_spec.precompiled_charsmap


def _tokenizer(vocab, normalizer, pre_tokenizer):
    from tokenizers import AddedToken, Tokenizer, models
    tok = Tokenizer(models.Unigram(vocab, unk_id=3, byte_fallback=False))
    tok.normalizer = normalizer
    tok.pre_tokenizer = pre_tokenizer
    tok.add_special_tokens([AddedToken(t, special=True) for t in SPECIALS])
    tok.add_tokens([AddedToken(t, special=True) for t in MARKERS])
    return tok


@pytest.fixture(scope="session")
def deberta_tok(spm_parts):
    """The checkpoint's shape of tokenizer.json (DebertaV2Converter)."""
    from tokenizers import Regex, normalizers, pre_tokenizers
    vocab, charsmap = spm_parts
    return _tokenizer(vocab, normalizers.Sequence([normalizers.Strip(), normalizers.Precompiled(charsmap),
                                                   normalizers.Replace(Regex(" {2,}"), " ")]),
                      pre_tokenizers.Sequence([pre_tokenizers.Metaspace(replacement="▁",
                                                                        prepend_scheme="always")]))


@pytest.fixture(scope="session")
def tok_dir(deberta_tok, tmp_path_factory):
    d = tmp_path_factory.mktemp("tok")
    (d / "tokenizer.json").write_text(deberta_tok.to_str(), encoding="utf-8")
    (d / "tokenizer_config.json").write_text(json.dumps({"tokenizer_class": "DebertaV2Tokenizer"}))
    return d


class Handle:
    """Direct C-ABI access (no Python wrapper)."""

    def __init__(self, tokenizer_json: str):
        self.lib = F.lib()
        self.h = C.c_void_p()
        b = tokenizer_json.encode()
        F.check(self.lib.gd_frontend_create(C.byref(self.h), b, len(b)))

    def encode(self, text: str):
        b = text.encode()
        cap = 8 * len(b) + 64
        buf = (C.c_int32 * cap)()
        n = C.c_int64()
        F.check(self.lib.gd_frontend_encode(self.h, b, len(b), buf, cap, C.byref(n)))
        return list(buf[:n.value])

    def __del__(self):
        self.lib.gd_frontend_destroy(self.h)


def _fuzz(vocab, seed, count, extra=()):
    import random
    r = random.Random(seed)
    pool = [p.replace("▁", " ") for p, _ in vocab[5:]]
    pool = r.sample(pool, min(300, len(pool))) + list("abcxyzABC  .,!?'`\"-_()0123") + EXOTIC + list(extra)
    out = []
    for _ in range(count):
        s = "".join(r.choice(pool) for _ in range(r.randint(0, 14)))
        if not any(t in s for t in SPECIALS + MARKERS):
            out.append(s)
    return out


def _assert_same_ids(tok, strings):
    h = Handle(tok.to_str())
    bad = [(s, h.encode(s), tok.encode(s, add_special_tokens=False).ids) for s in strings]
    bad = [b for b in bad if b[1] != b[2]]
    assert not bad, bad[:5]


def test_library_exports_every_declared_symbol():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = set(re.findall(r"^\s*(?:const\s+)?(?:int|void|char\s*\*)\s*\**\s*(gd_frontend_\w+)\s*\(", text, flags=re.M))
    assert len(names) >= 9
    lib = F.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert names == set(F._SIGNATURES)


def test_deberta_pipeline_matches_hf(deberta_tok, spm_parts):
    _assert_same_ids(deberta_tok, _fuzz(spm_parts[0], 0, 6000))
    # whole sentences of the training distribution, with odd spacing
    lines = _corpus(7, 500)
    _assert_same_ids(deberta_tok, lines + ["  " + s.replace(" ", "   ") + " \t" for s in lines[:100]])


def test_normalizer_and_pre_tokenizer_forms_match_hf(spm_parts):
    from tokenizers import Regex, normalizers, pre_tokenizers
    vocab, charsmap = spm_parts
    variants = [
        (normalizers.Sequence([normalizers.Lowercase(), normalizers.Strip(left=False), normalizers.NFKC(),
                               normalizers.Replace("``", '"'), normalizers.Replace(Regex("a+"), "A")]),
         pre_tokenizers.Metaspace(replacement="▁", prepend_scheme="always", split=False)),
        (normalizers.Sequence([normalizers.NFD(), normalizers.Strip(right=False), normalizers.Precompiled(charsmap)]),
         pre_tokenizers.Metaspace(replacement="▁", prepend_scheme="never")),
        (normalizers.Sequence([normalizers.NFC(), normalizers.NFKD(), normalizers.Replace(Regex("x{3,}"), "")]),
         pre_tokenizers.Sequence([pre_tokenizers.WhitespaceSplit(),
                                  pre_tokenizers.Metaspace(replacement="_", prepend_scheme="always")])),
        (None, None),
    ]
    for i, (norm, pre) in enumerate(variants):
        _assert_same_ids(_tokenizer(vocab, norm, pre), _fuzz(vocab, 10 + i, 2500, extra=["xxx", "aaa", "``"]))


def test_word_level_model_matches_hf():
    from tokenizers import Tokenizer, models, pre_tokenizers
    vocab = {t: i for i, t in enumerate(SPECIALS + ["hello", "world", "a", "b", ".", "東京", "é"])}
    tok = Tokenizer(models.WordLevel(vocab, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    words = ["hello", "world", "a", "b", ".", "東京", "é", "zz", " ", "　", "\t\n"]
    r = np.random.default_rng(3)
    _assert_same_ids(tok, ["".join(r.choice(words, size=int(r.integers(0, 8)))) for _ in range(500)])


def _hand_tokenizer(vocab, unk_id=0):
    return json.dumps({
        "normalizer": None, "pre_tokenizer": {"type": "Metaspace", "replacement": "▁",
                                              "prepend_scheme": "always", "split": True},
        "model": {"type": "Unigram", "unk_id": unk_id, "vocab": vocab, "byte_fallback": False},
        "added_tokens": []})


def test_viterbi_on_hand_scored_vocabulary():
    """Scores chosen so the best path is known: "▁abc" splits as
    ▁a + bc (-1 - 1 = -2 beats ▁ab + c = -1.5 - 1 and every
    single-character path); an unknown run "qq" is one fused [UNK]; on a tie
    the first candidate (the path whose last piece is shorter... found first)
    is kept."""
    vocab = [["[UNK]", 0.0], ["▁", -3.0], ["▁a", -1.0], ["▁ab", -1.5], ["bc", -1.0], ["a", -2.0],
             ["b", -2.0], ["c", -1.0]]
    h = Handle(_hand_tokenizer(vocab))
    assert h.encode("abc") == [2, 4]
    assert h.encode("abqqc") == [3, 0, 7]  # ▁ab, [UNK] for "qq", c
    assert h.encode("q") == [1, 0]  # ▁ then the unknown q
    # tie: "▁ab" (-1.5) against "▁a" + "b" (-1 - 2 = -3) is no tie; make one:
    tie = [["[UNK]", 0.0], ["▁", -1.0], ["x", -1.0], ["▁x", -2.0]]
    # "▁x": paths ▁ + x (-2, ends at x found second) and ▁x (-2, found first at position 0)
    assert Handle(_hand_tokenizer(tie)).encode("x") == [3]


def test_split_words_icu_matches_python_restatement(tok_dir):
    fe = NativeDecisionTokenizer(tok_dir)
    r = np.random.default_rng(5)
    pool = ["http://a.b/c?d=1", "https://x.y", "www.site.org", "me@mail.com", "a.b@c-d.io", "@user_1", "@", "co-op",
            "snake_case", "re-", "_x", "A", "b", "Z", "0", "9", ".", "!", "?", ",", "'", '"', "(", ")", "-", "_",
            " ", "  ", "\t", "\n", "　", " ", "é", "ΣΑΣ", "İ", "ǅ", "ß", "東京", "́", "‍",
            "‌", "\U0001f44d", "٠", "²", "Ⅳ", "ſ", "K", "؀", "‿", "ı", "HTTPS://Q.R", "WwW.x", "ſ@k.KK", "ﬃ", "ǅ", "İ"]
    texts = ["".join(r.choice(pool, size=int(r.integers(0, 10)))) for _ in range(3000)]
    texts += ["", ".", "end!", "why?", "x؀.", "ΟΔΟΣ", "ΟΔΟΣ.", "İstanbul"]
    bad = [(t, fe.split_words(t), split_words(t)) for t in texts]
    bad = [b for b in bad if b[1] != b[2]]
    assert not bad, bad[:5]


def test_split_words_swift_semantics(tok_dir):
    fe = NativeDecisionTokenizer(tok_dir)
    # per-scalar lower case: no final-sigma form, full mappings kept
    assert fe.split_words("ΟΔΟΣ") == ["οδοσ", "."]
    assert fe.split_words("İ") == ["i̇", "."]
    # a Prepend character joins the final '.', so Swift's last Character is not "."
    assert fe.split_words("x؀.") == ["x", "؀", ".", "."]
    assert fe.split_words("") == ["."]
    assert fe.split_words("Visit https://x.y/z now, mail a@b.co or @Bob_2!") == \
        ["visit", "https://x.y/z", "now", ",", "mail", "a@b.co", "or", "@bob_2", "!"]


def _random_tasks(r, words):
    tasks = []
    for t in range(int(r.integers(1, 4))):
        labels = [" ".join(r.choice(words, size=int(r.integers(1, 3)))) for _ in range(int(r.integers(1, 6)))]
        desc = None
        if r.random() < 0.5:
            desc = {lab: " ".join(r.choice(words, size=3)) for lab in labels if r.random() < 0.6}
            desc["not a label"] = "ignored"
        prompt = " ".join(r.choice(words, size=4)) if r.random() < 0.5 else None
        tasks.append(DecisionTask(f"task {t} {r.choice(words)}", tuple(labels), bool(r.random() < 0.5), prompt, desc))
    return tasks


def test_make_input_matches_hf_frontend(tok_dir, deberta_tok):
    native = NativeDecisionTokenizer(tok_dir)
    hf = NativeDecisionTokenizer(tok_dir, backend="hf")
    assert native.backend == "native" and hf.backend == "hf"
    assert native.pad_token_id == hf.pad_token_id == 0 and native.special_ids == hf.special_ids
    r = np.random.default_rng(11)
    words = ["kare", "motion", "Prestly", "東京", "é", "[L]", "(x)", "a-b", "www.q.io", "@me", "Ünï", "ﬁne", "  ",
             "[DESCRIPTION]", "zzq", "ΣΑΣ", "́", "\U0001f44d\U0001f3fd", "\r\n", "[SEP_TEXT]x"]
    for _ in range(300):
        tasks = _random_tasks(r, words)
        text = " ".join(r.choice(words, size=int(r.integers(0, 40))))
        buckets = [32, 64, 96, 128, 256, 512]
        try:
            want = hf.make_input(text, tasks, buckets)
        except TokenizerError as e:
            with pytest.raises(TokenizerError, match="does not fit"):
                native.make_input(text, tasks, buckets)
            assert "does not fit" in str(e)
            continue
        got = native.make_input(text, tasks, buckets)
        for k in ("input_ids", "attention_mask", "marker_indices", "marker_mask"):
            a, b = getattr(got, k), getattr(want, k)
            assert a.dtype == b.dtype and a.shape == b.shape, k
            np.testing.assert_array_equal(a, b, err_msg=k)
        assert native.encode_ids(text, tasks) == hf.encode_ids(text, tasks)


def test_entry_cache_and_clear(tok_dir):
    fe = NativeDecisionTokenizer(tok_dir)
    ids = []
    fe.append_tokenized("kare [L] motion", ids)
    again = []
    fe.clear_cache()
    fe.append_tokenized("kare [L] motion", again)
    assert ids == again and fe.special_ids["[L]"] in ids


def test_errors(tmp_path, deberta_tok):
    with pytest.raises(TokenizerError, match="missing tokenizer.json/tokenizer_config.json"):
        NativeDecisionTokenizer(tmp_path)
    (tmp_path / "tokenizer.json").write_text(deberta_tok.to_str(), encoding="utf-8")
    (tmp_path / "tokenizer_config.json").write_text("[1, 2")
    with pytest.raises(TokenizerError, match="Could not decode tokenizer_config.json"):
        NativeDecisionTokenizer(tmp_path)
    (tmp_path / "tokenizer_config.json").write_text("{}")
    fe = NativeDecisionTokenizer(tmp_path)
    task = DecisionTask("t", ("a", "b"))
    with pytest.raises(TokenizerError, match="at least one label"):
        fe.make_input("x", [])
    with pytest.raises(TokenizerError, match="at least one label"):
        fe.make_input("x", [task, DecisionTask("e", ())])
    with pytest.raises(TokenizerError, match=r"does not fit any requested bucket: \[\]"):
        fe.make_input("x", [task], [])
    with pytest.raises(TokenizerError, match=r"does not fit any requested bucket: \[8\]"):
        fe.make_input("a long text " * 20, [task], [8, 8])
    # C-ABI: bad UTF-8, small buffers (the needed size still reported), unsupported components
    h = Handle(deberta_tok.to_str())
    n = C.c_int64()
    assert h.lib.gd_frontend_encode(h.h, b"\xff\xfe", 2, None, 0, C.byref(n)) == -1
    assert h.lib.gd_frontend_encode(h.h, b"kare motion", 11, None, 0, C.byref(n)) == F.GD_ERR_SHAPE and n.value > 0
    bad = json.loads(deberta_tok.to_str())
    bad["model"] = {"type": "BPE", "vocab": {}, "merges": []}
    hh = C.c_void_p()
    b = json.dumps(bad).encode()
    assert h.lib.gd_frontend_create(C.byref(hh), b, len(b)) == -3
    assert b"BPE" in h.lib.gd_frontend_last_error()
    bad = json.loads(deberta_tok.to_str())
    bad["normalizer"]["normalizers"][2]["pattern"] = {"Regex": "[ab]+"}
    b = json.dumps(bad).encode()
    assert h.lib.gd_frontend_create(C.byref(hh), b, len(b)) == -3
    assert h.lib.gd_frontend_create(C.byref(hh), b"{", 1) == -8


def test_serving_frontend_is_native_and_matches_hf():
    from gliner_decide.synthetic import serving_examples, word_level_frontend, word_level_tokenizer_json
    from gliner_decide.frontend import tasks_from_json
    fe = word_level_frontend()
    assert fe.backend == "native"
    ref = NativeDecisionTokenizer.from_json(json.dumps(word_level_tokenizer_json()), backend="hf")
    assert ref.backend == "hf" and ref.special_ids == fe.special_ids
    for e in serving_examples(count=200):
        tasks = tasks_from_json(e["tasks"])
        a, b = fe.make_input(e["text"], tasks), ref.make_input(e["text"], tasks)
        np.testing.assert_array_equal(a.input_ids, b.input_ids)
        np.testing.assert_array_equal(a.marker_indices, b.marker_indices)
