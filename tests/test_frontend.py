"""Schema formatter, tokenizer front end and JSONL runner (no GPU).

The formatter follows NativeTokenizer.swift:76-212 and the runner
RawCLI.swift:104-223.  Expected id sequences are written out by hand from
the reference's schema layout with a word-level tokenizer (every
whitespace-separated piece is one id), so a dropped marker, a misplaced
separator or a wrong marker position shows as a different sequence; the
special-token cut is checked against a direct restatement of the reference's
scan loop on adversarial overlaps.
"""

import json

import numpy as np
import pytest

from gliner_decide.decode import DecisionTask
from gliner_decide.frontend import NativeDecisionTokenizer, TokenizerError, split_words, tasks_from_json
from gliner_decide import raw_cli

SPECIALS = ["[PAD]", "[CLS]", "[SEP]", "[UNK]", "[MASK]", "[P]", "[L]", "[SEP_STRUCT]", "[SEP_TEXT]",
            "[DESCRIPTION]"]
WORDS = ["(", ")", ":", ".", "!", "?", ",", "intent", "intent:", "what", "buy", "buy:", "sell", "hold",
         "purchase", "hello", "world", "sentiment", "sentiment:", "tone", "pos", "neg", "a", "b", "c"]


def word_level():
    """Word-level tokenizer: ids 0..9 are the specials, then WORDS; pieces are
    whitespace-separated; unknown pieces map to [UNK] = 3."""
    from tokenizers import Tokenizer, models, pre_tokenizers
    vocab = {t: i for i, t in enumerate(SPECIALS + WORDS)}
    tok = Tokenizer(models.WordLevel(vocab, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tok.add_special_tokens(SPECIALS)
    return tok, vocab


def frontend():
    tok, vocab = word_level()
    return NativeDecisionTokenizer.from_tokenizer(tok, {s: vocab[s] for s in SPECIALS}), vocab


def test_split_words_rules():
    # NativeTokenizer.swift:193-208: trailing "." unless . ! ?; URLs, e-mails
    # and @handles whole; hyphen/underscore compounds whole; lower case.
    assert split_words("Hello World") == ["hello", "world", "."]
    assert split_words("Why?") == ["why", "?"]
    assert split_words("Stop!") == ["stop", "!"]
    assert split_words("") == ["."]
    assert split_words("See https://Example.com/a?b=1 now") == ["see", "https://example.com/a?b=1", "now", "."]
    assert split_words("mail Bob.Smith@EXAMPLE.org or @Team_1.") == [
        "mail", "bob.smith@example.org", "or", "@team_1", "."]
    assert split_words("state-of-the-art under_score x--y") == [
        "state-of-the-art", "under_score", "x", "-", "-", "y", "."]
    assert split_words("www.site.io, ok") == ["www.site.io,", "ok", "."]
    # ICU \w includes combining marks (Python's \w does not): "e" + U+0301
    assert split_words("cafe\u0301 bar") == ["cafe\u0301", "bar", "."]
    assert split_words("a\tb\u00a0c") == ["a", "b", "c", "."]  # U+00A0 is \p{Z}


def test_schema_ids_one_task_by_hand():
    fe, v = frontend()
    task = DecisionTask("intent", ("buy", "sell"), prompt="what", label_descriptions={"buy": "purchase"})
    inp = fe.make_input("Hello world", [task])
    # ( [P] "intent: what [DESCRIPTION] buy: purchase" ( [L] buy [L] sell ) ) [SEP_TEXT] hello world .
    want = [v["("], v["[P]"], v["intent:"], v["what"], v["[DESCRIPTION]"], v["buy:"], v["purchase"], v["("],
            v["[L]"], v["buy"], v["[L]"], v["sell"], v[")"], v[")"], v["[SEP_TEXT]"], v["hello"], v["world"], v["."]]
    n = len(want)
    assert inp.input_ids.shape == (1, 32) and inp.input_ids.dtype == np.int32
    assert inp.input_ids[0, :n].tolist() == want and np.all(inp.input_ids[0, n:] == v["[PAD]"])
    assert inp.attention_mask.dtype == np.float16 and inp.attention_mask[0].tolist() == [1.0] * n + [0.0] * (32 - n)
    assert inp.marker_indices.tolist() == [[[8, 10]]] and inp.marker_mask.tolist() == [[[1.0, 1.0]]]
    assert inp.marker_mask.dtype == np.float32


def test_schema_two_tasks_ragged_labels():
    fe, v = frontend()
    tasks = [DecisionTask("intent", ("buy", "sell", "hold")), DecisionTask("sentiment", ("pos", "neg"), True)]
    inp = fe.make_input("a b c!", tasks)
    want = [v["("], v["[P]"], v["intent"], v["("], v["[L]"], v["buy"], v["[L]"], v["sell"], v["[L]"], v["hold"],
            v[")"], v[")"], v["[SEP_STRUCT]"],
            v["("], v["[P]"], v["sentiment"], v["("], v["[L]"], v["pos"], v["[L]"], v["neg"], v[")"], v[")"],
            v["[SEP_TEXT]"], v["a"], v["b"], v["c"], v["!"]]
    assert inp.input_ids[0, :len(want)].tolist() == want
    assert inp.marker_indices.shape == (1, 2, 3)
    assert inp.marker_indices.tolist() == [[[4, 6, 8], [17, 19, 0]]]
    assert inp.marker_mask.tolist() == [[[1, 1, 1], [1, 1, 0]]]


def test_buckets_and_errors():
    fe, v = frontend()
    task = DecisionTask("intent", ("buy",))
    # 9 schema ids + [SEP_TEXT] + words + "."
    short = fe.make_input("hello", [task])
    assert short.shape == (1, 32, 1, 1)
    long_text = " ".join(["hello"] * 40)
    assert fe.make_input(long_text, [task]).shape[1] == 64
    assert fe.make_input(long_text, [task], buckets=[512, 96, 96]).shape[1] == 96
    with pytest.raises(TokenizerError, match="does not fit"):
        fe.make_input(long_text, [task], buckets=[32])
    with pytest.raises(TokenizerError, match="does not fit"):
        fe.make_input("hello", [task], buckets=[])
    with pytest.raises(TokenizerError, match="at least one label"):
        fe.make_input("hello", [])
    with pytest.raises(TokenizerError, match="at least one label"):
        fe.make_input("hello", [task, DecisionTask("empty", ())])
    # unknown words map to [UNK]
    assert fe.make_input("zzz", [task]).input_ids[0, 9] == v["[UNK]"]


def _reference_cut(text, specials):
    """NativeTokenizer.swift:159-182 restated as the loop it is: at each
    cursor take the earliest occurrence of any special token, the longer one
    on equal starts; plain text between goes to the tokenizer."""
    out, cursor = [], 0
    while cursor < len(text):
        best = None
        for tok in specials:
            i = text.find(tok, cursor) if tok else -1
            if i < 0:
                continue
            if best is None or i < best[0] or (i == best[0] and len(tok) > len(best[1])):
                best = (i, tok)
        if best is None:
            out.append(("plain", text[cursor:]))
            break
        if best[0] > cursor:
            out.append(("plain", text[cursor:best[0]]))
        out.append(("special", best[1]))
        cursor = best[0] + len(best[1])
    return out


def test_special_token_cut_matches_reference_loop():
    from tokenizers import Regex, Tokenizer, models, pre_tokenizers
    specials = {"<a>": 100, "<a><b>": 101, "<b>": 102, "ab": 103, "b": 104, "": 105}
    vocab = {c: i for i, c in enumerate("xyz<>ab")}
    vocab["[UNK]"] = 99
    tok = Tokenizer(models.WordLevel(vocab, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.Split(Regex("."), "isolated")
    fe = NativeDecisionTokenizer.from_tokenizer(tok, specials)
    r = np.random.default_rng(0)
    alphabet = list("xyz<>ab")
    for _ in range(300):
        text = "".join(r.choice(alphabet, size=int(r.integers(0, 14))))
        want = []
        for kind, s in _reference_cut(text, list(specials)):
            if kind == "special":
                want.append(specials[s])
            else:
                want += tok.encode(s, add_special_tokens=False).ids
        got = []
        fe.append_tokenized(text, got)
        assert got == want, text


def test_directory_loader(tmp_path):
    tok, vocab = word_level()
    (tmp_path / "tokenizer.json").write_text(tok.to_str())
    with pytest.raises(TokenizerError, match="missing"):
        NativeDecisionTokenizer(tmp_path)
    (tmp_path / "tokenizer_config.json").write_text("{not json")
    with pytest.raises(TokenizerError, match="tokenizer_config"):
        NativeDecisionTokenizer(tmp_path)
    (tmp_path / "tokenizer_config.json").write_text(json.dumps({"tokenizer_class": "DebertaV2Tokenizer"}))
    fe = NativeDecisionTokenizer(tmp_path)
    assert fe.special_ids["[SEP_TEXT]"] == vocab["[SEP_TEXT]"] and fe.pad_token_id == 0
    ref, _ = frontend()
    task = DecisionTask("intent", ("buy", "sell"))
    np.testing.assert_array_equal(fe.make_input("hello world", [task]).input_ids,
                                  ref.make_input("hello world", [task]).input_ids)


def test_unigram_entries_tokenized_one_by_one():
    """With the checkpoint's kind of tokenizer (Unigram + Metaspace) every
    schema entry and word is encoded on its own: the ids are the concatenation
    of the per-entry encodings (each gets its own leading '▁')."""
    from tokenizers import Tokenizer, models, pre_tokenizers
    pieces = [("[PAD]", 0.0), ("[CLS]", 0.0), ("[SEP]", 0.0), ("[UNK]", 0.0), ("▁", -2.0), ("▁(", -1.0),
              ("▁)", -1.0), ("▁hello", -1.0), ("▁world", -1.5), ("▁.", -1.0), ("▁intent", -1.0), ("▁buy", -1.0),
              ("▁sell", -1.0), (":", -1.0)] + [(c, -5.0) for c in "abcdefghijklmnopqrstuvwxyz.:()"]
    tok = Tokenizer(models.Unigram(pieces, unk_id=3, byte_fallback=False))
    tok.pre_tokenizer = pre_tokenizers.Metaspace(replacement="▁", prepend_scheme="always")
    sp = ["[P]", "[L]", "[SEP_STRUCT]", "[SEP_TEXT]", "[DESCRIPTION]"]
    tok.add_special_tokens(["[PAD]", "[CLS]", "[SEP]", "[UNK]"] + sp)
    special_ids = {s: tok.token_to_id(s) for s in ["[PAD]", "[CLS]", "[SEP]", "[UNK]"] + sp}
    fe = NativeDecisionTokenizer.from_tokenizer(tok, special_ids)
    task = DecisionTask("intent", ("buy", "sell"))
    ids, markers = fe.encode_ids("Hello world", [task])
    enc = lambda s: tok.encode(s, add_special_tokens=False).ids  # noqa: E731
    want = (enc("(") + [special_ids["[P]"]] + enc("intent") + enc("(") + [special_ids["[L]"]] + enc("buy")
            + [special_ids["[L]"]] + enc("sell") + enc(")") + enc(")") + [special_ids["[SEP_TEXT]"]]
            + enc("hello") + enc("world") + enc("."))
    assert ids == want
    assert enc("(") == [tok.token_to_id("▁(")] and enc("hello") == [tok.token_to_id("▁hello")]
    assert len(ids) == 14 and markers == [[4, 6]]


def test_task_json_strictness():
    t = tasks_from_json({"tasks": [{"name": "a", "labels": ["x", "y"], "multiLabel": True, "prompt": "p",
                                    "labelDescriptions": {"x": "ex"}}]})
    assert t == [DecisionTask("a", ("x", "y"), True, "p", {"x": "ex"})]
    assert DecisionTask.from_json(t[0].to_json()) == t[0]
    for bad in ({"labels": ["x"], "multiLabel": False}, {"name": "a", "multiLabel": False},
                {"name": "a", "labels": ["x"]}, {"name": "a", "labels": "x", "multiLabel": False},
                {"name": "a", "labels": ["x"], "multiLabel": 1}, {"name": 3, "labels": ["x"], "multiLabel": False}):
        with pytest.raises(ValueError):
            tasks_from_json([bad])


class _FakeModel:
    """Stands in for the classifier in host-only runner tests: logits are a
    fixed function of each row's own ids and markers (so a row's decision
    does not depend on its batch), and every call is recorded."""

    def __init__(self):
        self.calls = []

    def classify(self, inp):
        from gliner_decide.classifier import InferenceResult
        ids = np.asarray(inp.input_ids).astype(np.float64)
        mk = np.asarray(inp.marker_indices)
        B, L, Hh, O = inp.shape
        self.calls.append((B, L, Hh, O))
        logits = np.empty((B, Hh, O), np.float32)
        for b in range(B):
            for h in range(Hh):
                for o in range(O):
                    logits[b, h, o] = np.sin(ids[b].sum() * 0.37 + 1.3 * h + 0.7 * o + 0.01 * mk[b, h, o])
        logits[np.asarray(inp.marker_mask) == 0] = -10000.0
        return InferenceResult(logits, 1_000_000 * B, [])


def _examples(n, seed=0):
    r = np.random.default_rng(seed)
    words = ["hello", "world", "buy", "sell", "a", "b", "c", "zzz"]
    out = []
    for i in range(n):
        length = int(r.integers(1, 60))
        text = " ".join(r.choice(words, size=length))
        ntask = int(r.integers(1, 3))
        tasks = [{"name": "intent", "labels": ["buy", "sell", "hold"][:int(r.integers(1, 4))],
                  "multiLabel": bool(r.integers(0, 2))} for _ in range(ntask)]
        out.append({"id": f"ex{i}", "text": text, "tasks": tasks})
    return out


def _check_rows_match_alone(fe, exs, res):
    """Every row decoded with its own tasks, equal to running it alone."""
    from gliner_decide.decode import decode
    alone = _FakeModel()
    for e, r in zip(exs, res):
        tasks = tasks_from_json(e["tasks"])
        one = alone.classify(fe.make_input(e["text"], tasks))
        assert r["predictions"] == [p.to_json() for p in decode(one.logits, 0, tasks)]
        assert [p["task"] for p in r["predictions"]] == [t.name for t in tasks]
        assert r["inferenceMilliseconds"] == pytest.approx(1.0) and r["preprocessingMilliseconds"] >= 0


def test_jsonl_runner_reference_grouping(tmp_path):
    """group_by_length=False: the batches of RawCLI.swift:135-150, rows grouped
    by (L, Hh, O) in input order, each group in runs of the batch size."""
    fe, _ = frontend()
    exs = _examples(70)
    model = _FakeModel()
    res = raw_cli.run_examples(raw_cli.parse_jsonl("\n".join(json.dumps(e) for e in exs)), fe, model,
                               batch_size=8, group_by_length=False)
    assert [r["id"] for r in res] == [e["id"] for e in exs]
    shapes = {}
    for e in exs:
        k = fe.make_input(e["text"], tasks_from_json(e["tasks"])).shape[1:]
        shapes[k] = shapes.get(k, 0) + 1
    want_calls = sorted((min(8, n - s), *k) for k, n in shapes.items() for s in range(0, n, 8))
    assert sorted(model.calls) == want_calls
    _check_rows_match_alone(fe, exs, res)


def test_jsonl_runner_length_grouping_and_order(tmp_path):
    """Default: rows grouped by L only; each batch's markers padded to its
    largest Hh and O; decisions equal to running each row alone."""
    fe, _ = frontend()
    exs = _examples(70)
    path = tmp_path / "in.jsonl"
    path.write_text("\n".join(json.dumps(e) for e in exs) + "\n\n")
    model = _FakeModel()
    out = tmp_path / "out.json"
    logs = []
    res = raw_cli.run_jsonl(path, fe, model, batch_size=8, output=out, log=logs.append)
    assert json.loads(out.read_text()) == res
    assert [r["id"] for r in res] == [e["id"] for e in exs]
    assert logs[-1] == "tokenized 70/70" and "tokenized 0/70" not in logs
    by_len = {}
    for e in exs:
        inp = fe.make_input(e["text"], tasks_from_json(e["tasks"]))
        by_len.setdefault(inp.shape[1], []).append(inp.shape[2:])
    want_calls = []
    for L, shp in by_len.items():
        for s in range(0, len(shp), 8):
            part = shp[s:s + 8]
            want_calls.append((len(part), L, max(h for h, _ in part), max(o for _, o in part)))
    assert sorted(model.calls) == sorted(want_calls)
    _check_rows_match_alone(fe, exs, res)


def test_jsonl_errors_name_the_line(tmp_path):
    fe, _ = frontend()
    p = tmp_path / "bad.jsonl"
    p.write_text(json.dumps(_examples(1)[0]) + "\n" + json.dumps({"id": "x", "text": "t"}) + "\n")
    with pytest.raises(ValueError, match="line 2"):
        raw_cli.run_jsonl(p, fe, _FakeModel())
    p.write_text("{oops\n")
    with pytest.raises(ValueError, match="line 1"):
        raw_cli.run_jsonl(p, fe, _FakeModel())
    with pytest.raises(ValueError):
        raw_cli.run_examples([], fe, _FakeModel(), batch_size=0)


def test_single_mode_and_options(tmp_path, capsys):
    import io
    fe, _ = frontend()
    tasks = [DecisionTask("intent", ("buy", "sell"))]
    err = io.StringIO()
    dump = tmp_path / "in.safetensors"

    class Torchish(_FakeModel):
        def classify(self, inp):
            import torch
            r = super().classify(inp)
            r.logits = torch.from_numpy(r.logits)
            return r

    preds = raw_cli.run_single("hello world", tasks, fe, Torchish(), dump_input=dump, err=err)
    assert json.loads(capsys.readouterr().out) == preds and len(preds) == 1
    assert "preprocessing_ms:" in err.getvalue() and "inference_ms:" in err.getvalue()
    from gliner_decide.classifier import DecisionInput
    back = DecisionInput.from_safetensors(dump)
    np.testing.assert_array_equal(back.input_ids, fe.make_input("hello world", tasks).input_ids)
    a = raw_cli.parse_args(["--jsonl", "x.jsonl", "--buckets", "64,32,x,,128", "--batch-size", "4"])
    assert a.buckets == [64, 32, 128] and a.batch_size == 4 and a.weights.endswith(".safetensors")
    with pytest.raises(SystemExit):
        raw_cli.parse_args([])
