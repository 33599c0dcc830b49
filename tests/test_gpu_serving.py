"""The JSONL runner (RawCLI.swift:104-171) end to end on the HIP classifier:
text -> schema ids -> grouped batches -> logits -> decisions.

A row's decision must not depend on the batch it ran in: every example is
also run alone (batch of one, its own bucket) and in the reference's (L, Hh,
O) grouping besides the default length grouping, and the probabilities
agree within 1e-3 with identical label sets (a difference is accepted only
where the single-row decision is itself within 2e-3 of a tie).  Two examples
are recomputed by the oracle from the same ids.
"""

import json

import numpy as np
import pytest

from oracle import deberta as O

pytestmark = pytest.mark.gpu

VOCAB = 3000


def _tokenizer_json():
    """A WordLevel tokenizer.json: the specials as added tokens, 1000 words."""
    specials = ["[PAD]", "[CLS]", "[SEP]", "[UNK]", "[MASK]", "[P]", "[L]", "[SEP_STRUCT]", "[SEP_TEXT]",
                "[DESCRIPTION]"]
    vocab = {t: i for i, t in enumerate(specials)}
    for i in range(1000):
        vocab[f"w{i}"] = 1000 + i
    for j, t in enumerate(["(", ")", ".", ":", "intent", "tone", "topic", "a", "b", "c", "d", "e"]):
        vocab[t] = 100 + j
    added = [{"id": vocab[t], "content": t, "single_word": False, "lstrip": False, "rstrip": False,
              "normalized": False, "special": True} for t in specials]
    return json.dumps({"version": "1.0", "added_tokens": added, "normalizer": None,
                       "pre_tokenizer": {"type": "WhitespaceSplit"},
                       "model": {"type": "WordLevel", "vocab": vocab, "unk_token": "[UNK]"}})


def _frontend(backend="native"):
    """The C++ front end (the runner's default); backend="hf" for the check."""
    from gliner_decide.frontend import NativeDecisionTokenizer
    return NativeDecisionTokenizer.from_json(_tokenizer_json(), backend=backend)


def _examples(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        words = int(np.exp(r.uniform(np.log(4), np.log(440))))
        text = " ".join(f"w{int(x)}" for x in r.integers(0, 1000, size=words))
        tasks = []
        for name in ["intent", "tone", "topic"][:int(r.integers(1, 3))]:
            labels = list("abcde")[:int(r.integers(2, 6))]
            tasks.append({"name": name, "labels": labels, "multiLabel": bool(r.integers(0, 2))})
        out.append({"id": f"r{i}", "text": text, "tasks": tasks})
    return out


def _decision(pred):
    return pred["labels"], np.asarray(pred["probabilities"])


def _assert_same_decisions(got, want, tol=1e-3):
    for g, w in zip(got, want):
        (gl, gp), (wl, wp) = _decision(g), _decision(w)
        assert np.max(np.abs(gp - wp)) <= tol
        if gl != wl:
            srt = np.sort(wp)[::-1]
            margin = min(np.min(np.abs(wp - 0.5)), srt[0] - srt[1]) if len(srt) > 1 else 0.0
            assert margin <= 2 * tol, (gl, wl, margin)


def test_jsonl_runner_end_to_end(tmp_path):
    from gliner_decide import GLiNERDecideClassifier
    from gliner_decide import raw_cli
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=VOCAB)
    w = synthetic_weights(pc, seed=11)
    model = GLiNERDecideClassifier(w, pc, use_compiled_graph=True)
    fe = _frontend()
    assert fe.backend == "native"
    exs = _examples(96, seed=3)
    path = tmp_path / "in.jsonl"
    path.write_text("\n".join(json.dumps(e) for e in exs))
    out = tmp_path / "out.json"
    res = raw_cli.run_jsonl(path, fe, model, batch_size=8, output=out)
    assert json.loads(out.read_text()) == res and [r["id"] for r in res] == [e["id"] for e in exs]
    examples = raw_cli.parse_jsonl(path.read_text())
    lengths = set()
    hf = _frontend("hf")
    for ex, r in zip(examples, res):
        inp = fe.make_input(ex.text, ex.tasks)
        np.testing.assert_array_equal(inp.input_ids, hf.make_input(ex.text, ex.tasks).input_ids)
        lengths.add(inp.shape[1])
        alone = model.classify(inp).logits.float().cpu().numpy()
        from gliner_decide.decode import decode
        want = [p.to_json() for p in decode(alone, 0, ex.tasks)]
        _assert_same_decisions(r["predictions"], want)
        assert r["inferenceMilliseconds"] > 0
    assert lengths == {32, 64, 96, 128, 256, 512}
    # the reference's (L, Hh, O) grouping: other batches, the same decisions
    ref = raw_cli.run_examples(examples, fe, model, batch_size=8, group_by_length=False)
    for a, b in zip(ref, res):
        assert a["id"] == b["id"]
        _assert_same_decisions(a["predictions"], b["predictions"])
    # the oracle on two rows, from the ids the front end made
    oc = O.Config(**{k: getattr(pc, k) for k in O.Config.__dataclass_fields__})
    om = O.OracleModel(O.ModelWeights.from_store(w, oc), oc, dtype=np.float64)
    for i in (0, 1):
        ex = examples[i]
        inp = fe.make_input(ex.text, ex.tasks)
        logits = om.forward(np.asarray(inp.input_ids), np.asarray(inp.attention_mask),
                            np.asarray(inp.marker_indices), np.asarray(inp.marker_mask))
        tasks = [(len(t.labels), t.multi_label) for t in ex.tasks]
        for (sel, probs), pred in zip(O.decode(logits[0], tasks), res[i]["predictions"]):
            np.testing.assert_allclose(pred["probabilities"], probs, atol=1e-3)
