"""Host-side logic of the package (no GPU): decode, buckets, batch chunking,
configuration and the synthetic workloads."""

import math

import numpy as np
import pytest

from gliner_decide import DeBERTaV2Configuration, DecisionTask, decode, make_batch_chunk, select_bucket
from gliner_decide import synthetic as S
from oracle import deberta as O


def test_configuration_default():
    c = DeBERTaV2Configuration.default()
    assert (c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads, c.head_size) == (
        1024, 4096, 24, 16, 64)
    assert c.layer_norm_eps == 1e-7 and c.position_buckets == 256 and c.hidden_act == "gelu"


def test_decode_matches_oracle_and_rules():
    r = np.random.default_rng(0)
    logits = r.standard_normal((4, 2, 6)).astype(np.float32)
    tasks = [DecisionTask("a", tuple("uvwxyz"), False), DecisionTask("b", tuple("pqrs"), True)]
    for row in range(4):
        got = decode(logits, row, tasks)
        want = O.decode(logits[row], [(6, False), (4, True)])
        for p, (sel, probs) in zip(got, want):
            np.testing.assert_allclose(p.probabilities, probs, rtol=1e-12)
            assert len(p.labels) == len(sel)
    # multi-label: nothing >= 0.5 -> argmax fallback; ties -> first
    out = decode(np.array([[[-3.0, -1.0, -2.0]]]), 0, [DecisionTask("t", ("a", "b", "c"), True)])
    assert out[0].labels == ["b"]
    out = decode(np.array([[[1.0, 1.0]]]), 0, [DecisionTask("t", ("a", "b"), False)])
    assert out[0].labels == ["a"] and math.isclose(out[0].probabilities[0], 0.5)


def test_buckets_and_chunks():
    assert [select_bucket(n) for n in (1, 32, 33, 64, 65, 96, 97, 128, 129, 256, 257, 512)] == [
        32, 32, 64, 64, 96, 96, 128, 128, 256, 256, 512, 512]
    assert select_bucket(40, buckets=[256, 64, 64]) == 64
    with pytest.raises(ValueError):
        select_bucket(600)
    arrays = {"x": np.arange(12).reshape(6, 2)}
    chunk, valid = make_batch_chunk(arrays, 4, 6, 5)
    assert valid == 2 and chunk["x"].shape == (5, 2) and (chunk["x"][2:] == [10, 11]).all()
    chunk, valid = make_batch_chunk(arrays, 0, 4, 4)
    assert valid == 4 and chunk["x"].shape == (4, 2)


def test_bias_division_by_reciprocal_is_exact():
    """The attention kernel divides the fp16 bias sum by fp16(sqrt(192)) =
    13.859375 as a multiply by the fp32 reciprocal.  For every finite fp16
    numerator the fp16 result equals the correctly rounded quotient."""
    s = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    s = s[np.isfinite(s)]
    scale = np.float16(math.sqrt(192.0))
    assert float(scale) == 13.859375
    exact = (s.astype(np.float64) / float(scale)).astype(np.float16)
    recip = np.float32(1.0) / np.float32(scale)
    via_mul = (s.astype(np.float32) * recip).astype(np.float16)
    np.testing.assert_array_equal(via_mul.view(np.uint16), exact.view(np.uint16))


def test_synthetic_weights_are_subset_stable():
    cfg = DeBERTaV2Configuration(hidden_size=128, intermediate_size=256, num_hidden_layers=3, num_attention_heads=2,
                                 vocab_size=64, classifier_hidden=128)
    full = S.synthetic_weights(cfg, seed=3)
    one = S.synthetic_weights(cfg, seed=3, layers=[1])
    for k, v in one.items():
        np.testing.assert_array_equal(v, full[k])
    g = full["encoder.encoder.layer.0.output.LayerNorm.weight"].astype(np.float64)
    assert abs(g.mean() - 1) < 0.01 and 0.01 < g.std() < 0.03
    assert all(v.dtype == np.float16 for v in full.values())


def test_classification_workload_layout():
    b = S.classification_batch(seed=4)
    assert b.shape == (32, 256, 1, 5)
    lengths = b.attention_mask.sum(1)
    assert lengths.min() >= 40 and lengths.max() <= 256
    assert (b.input_ids[:, 0] == S.CLS_ID).all()
    assert (b.input_ids[np.arange(32), lengths.astype(int) - 1] == S.SEP_ID).all()
    assert (b.input_ids[:, 1:6] == S.LABEL_MARKER_ID).all()
    assert (b.input_ids[b.attention_mask == 0] == 0).all()


def test_long_context_workload_layout():
    b = S.long_context_batch(seed=6)
    assert b.shape == (64, 512, 3, 20) and (b.attention_mask == 1).all()
    assert b.marker_mask[:, 2].sum(1).tolist() == [8] * 64
    for row in range(64):
        for h in range(3):
            pos = b.marker_indices[row, h][b.marker_mask[row, h] > 0]
            assert (b.input_ids[row, pos] == S.LABEL_MARKER_ID).all()


def test_bucket_mix_workload():
    batches = S.bucket_mix(seed=5)
    assert sum(x.valid_rows for x in batches) == 4096
    for x in batches:
        B, L, Hh, O_ = x.shape
        assert B == 32 and L in (32, 64, 96, 128, 256, 512) and Hh <= 2 and O_ <= 10
        lengths = x.attention_mask.sum(1)
        assert lengths.max() <= L and (L == 32 or lengths[:x.valid_rows].max() > {64: 32, 96: 64, 128: 96, 256: 128,
                                                                                  512: 256}[L])
        # padded rows copy the last valid row (main.swift:22-49)
        if x.valid_rows < 32:
            assert (x.input_ids[x.valid_rows:] == x.input_ids[x.valid_rows - 1]).all()


def test_row_extents_definition():
    """decode.row_extents against the definition written as loops: the larger
    of (last unmasked position + 1) and (last position an unmasked marker slot
    reads + 1), out-of-range markers reading position 0."""
    from gliner_decide.decode import row_extents
    r = np.random.default_rng(3)
    for _ in range(50):
        B, L, S = int(r.integers(1, 6)), int(r.integers(1, 40)), int(r.integers(1, 6))
        mask = (r.random((B, L)) < r.random()).astype(np.float16)
        mi = r.integers(-3, L + 3, size=(B, 1, S)).astype(np.int32)
        mm = (r.random((B, 1, S)) < 0.6).astype(np.float32)
        want = []
        for b in range(B):
            e = 0
            for l in range(L):
                if mask[b, l] > 0:
                    e = l + 1
            for s in range(S):
                if mm[b, 0, s] > 0:
                    p = mi[b, 0, s] if 0 <= mi[b, 0, s] < L else 0
                    e = max(e, p + 1)
            want.append(e)
        assert row_extents(mask, mi, mm).tolist() == want


def test_prepare_weights_filters_and_casts(tmp_path):
    """Tools/prepare_model.py:82-113: encoder.* and classifier.* kept, floats
    cast to fp16 (round to nearest even), integers kept, other heads dropped,
    required tensors enforced, metadata written; bf16 sources read too."""
    import json
    import struct

    import torch
    from safetensors.torch import save_file
    from gliner_decide.prepare import REQUIRED, prepare_weights
    r = np.random.default_rng(0)
    src = {k: torch.from_numpy(r.standard_normal((4, 8)).astype(np.float32)) for k in REQUIRED}
    src["encoder.encoder.layer.0.output.dense.bias"] = torch.tensor([1 + 2 ** -11, 1 + 3 * 2 ** -11])
    src["encoder.embeddings.position_ids"] = torch.arange(5, dtype=torch.int64)
    src["span_rep.project.weight"] = torch.ones(3, 3)
    src["count_embed.weight"] = torch.ones(2)
    save_file(src, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text('{"model_type": "deberta-v2"}')
    out = prepare_weights(tmp_path / "model.safetensors", tmp_path / "out", tmp_path / "config.json")
    from safetensors.numpy import load_file
    got = load_file(str(out))
    assert set(got) == set(REQUIRED) | {"encoder.encoder.layer.0.output.dense.bias", "encoder.embeddings.position_ids"}
    assert got["classifier.0.weight"].dtype == np.float16 and got["encoder.embeddings.position_ids"].dtype == np.int64
    np.testing.assert_array_equal(got["classifier.0.weight"], src["classifier.0.weight"].numpy().astype(np.float16))
    # ties round to even: 1 + 2^-11 -> 1, 1 + 3 * 2^-11 -> 1 + 2^-9
    assert got["encoder.encoder.layer.0.output.dense.bias"].tolist() == [1.0, 1 + 2 ** -9]
    n = struct.unpack("<Q", out.read_bytes()[:8])[0]
    meta = json.loads(out.read_bytes()[8:8 + n])["__metadata__"]
    assert meta == {"source_model": "fastino/GLiNER2.5-Decide",
                    "source_revision": "65624f1a0265b3f612bae66a2685a06b94a68a9d",
                    "precision": "float16", "scope": "encoder+classification-only"}
    assert (tmp_path / "out" / "encoder-config.json").read_text() == '{"model_type": "deberta-v2"}'
    # bf16 source
    save_file({k: v.to(torch.bfloat16) for k, v in src.items() if v.is_floating_point()},
              str(tmp_path / "bf16.safetensors"))
    got16 = load_file(str(prepare_weights(tmp_path / "bf16.safetensors", tmp_path / "o2")))
    np.testing.assert_array_equal(got16["classifier.2.weight"],
                                  src["classifier.2.weight"].to(torch.bfloat16).float().numpy().astype(np.float16))
    del src["classifier.2.weight"]
    save_file(src, str(tmp_path / "partial.safetensors"))
    with pytest.raises(RuntimeError, match="missing required weights: \\['classifier.2.weight'\\]"):
        prepare_weights(tmp_path / "partial.safetensors", tmp_path / "o3")


def test_decode_multi_label_extreme_logits():
    """fp16 logits reach -65504: the sigmoid is 0 there (IEEE exp overflow to
    +inf, as Swift's Double exp), not an exception; the argmax fallback still
    picks the largest."""
    logits = np.array([[[-800.0, 3.0, -65504.0]], [[-65504.0, -900.0, -1000.0]]], np.float32)
    tasks = [DecisionTask("m", ("a", "b", "c"), True)]
    p0 = decode(logits, 0, tasks)[0]
    assert p0.labels == ["b"] and p0.probabilities[0] == 0.0 and p0.probabilities[2] == 0.0
    p1 = decode(logits, 1, tasks)[0]
    assert p1.probabilities == [0.0, 0.0, 0.0] and p1.labels == ["a"]  # first of equal maxima
