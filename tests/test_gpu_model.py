"""GPU parity of the classifier context (layers, encoder, head, decode) against
the oracle, through the C-ABI.

Bars: hidden states within 2e-3 max-abs where the fp16 grid allows it
(|h| < 2, ulp <= 9.8e-4) and within 2 fp16 ulp elsewhere (for |h| >= 4 a
single ulp is 3.9e-3 > 2e-3, so no fp16 implementation can promise 2e-3
there); label probabilities within 1e-3; identical argmax and thresholded
label sets, without exception (heads whose reference decision lies within
2e-3 of a tie are counted and printed).  The large workloads are checked
whole against the batched torch restatement with the same fp16 rounding
points (oracle/torch_cpu.py, round16=True) and on chosen rows against the
float64 oracle.
"""

import numpy as np
import pytest
import torch

from oracle import deberta as O

pytestmark = pytest.mark.gpu


def _models(cfg_kwargs, seed, rows_limit=None):
    from gliner_decide import GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    pc = DeBERTaV2Configuration(**cfg_kwargs)
    w = synthetic_weights(pc, seed=seed)
    oc = O.Config(**{k: getattr(pc, k) for k in O.Config.__dataclass_fields__})
    gpu = GLiNERDecideClassifier(w, pc)
    return gpu, w, pc, oc


def assert_hidden_close(got, want):
    diff = np.abs(got - want)
    small = np.abs(want) < 2.0
    assert diff[small].max(initial=0) <= 2e-3, f"max diff {diff[small].max():.3g} on |h| < 2"
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14))) - 10)
    assert np.all(diff <= np.maximum(2e-3, 2 * ulp)), f"max diff {diff.max():.3g}"


def test_single_layer_workload():
    """One layer, B=1, L=32, all-ones mask, hidden ~ N(0,1), weights ~ N(0,0.02)."""
    from gliner_decide.synthetic import layer_inputs
    gpu, w, pc, oc = _models(dict(num_hidden_layers=1, vocab_size=1024), seed=1)
    d = layer_inputs(seed=1)
    out = gpu.layer_forward(0, torch.from_numpy(d["hidden"]).cuda(), torch.from_numpy(d["mask"]).cuda())
    got = out.float().cpu().numpy()
    mw = O.ModelWeights.from_store(w, oc)
    pq, pk = O.relative_tables(mw, oc)[0]
    want = O.encoder_layer(d["hidden"], mw.layers[0], pq, pk, d["mask"], oc)
    assert_hidden_close(got, want)


def test_encoder_and_logits_small_model_padded():
    gpu, w, pc, oc = _models(dict(num_hidden_layers=2, vocab_size=3000), seed=9)
    r = np.random.default_rng(2)
    B, L = 3, 64
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    lengths = np.array([64, 40, 17])
    mask = (np.arange(L)[None] < lengths[:, None]).astype(np.float16)
    ids[mask == 0] = 0
    mi = np.array([[[1, 2, 3, 4], [5, 6, 0, 0]]] * B, np.int32)
    mm = np.array([[[1, 1, 1, 1], [1, 1, 0, 0]]] * B, np.float32)
    from gliner_decide import DecisionInput
    inp = DecisionInput(ids, mask, mi, mm)
    res = gpu.classify(inp)
    hid = gpu.encode(inp).float().cpu().numpy()
    om = O.OracleModel(O.ModelWeights.from_store(w, oc), oc)
    want_h = om.encode(ids, mask)
    # Two layers of fp16 intermediates: bound the GPU by the spread between two
    # valid restatements of the same rounding points (float64 vs float32
    # accumulation), with a factor 2 and the 2e-3 floor.
    om32 = O.OracleModel(O.ModelWeights.from_store(w, oc), oc, dtype=np.float32)
    floor = np.max(np.abs(om32.encode(ids, mask).astype(np.float64) - want_h))
    err = np.max(np.abs(hid - want_h))  # padded query rows included (key-only masking)
    assert err <= max(2e-3, 2 * floor), (err, floor)
    want_logits = O.classifier_head(want_h, mi, mm, om.w)
    got_logits = res.logits.float().cpu().numpy()
    assert np.all(got_logits[mm == 0] == -10000.0)
    assert np.max(np.abs(got_logits - want_logits)) <= 2e-3


def _extent_batch(L, seed, B=6):
    """Rows of different lengths, a marker past the row's last unmasked
    token, an all-masked row, a mask with holes, a one-token row, and a
    masked marker slot pointing past the extent."""
    r = np.random.default_rng(seed)
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    lengths = np.array([L, 40, 17, 0, L // 2 + 3, 1])[:B]
    mask = (np.arange(L)[None] < lengths[:, None]).astype(np.float16)
    mask[4, 20:30] = 0  # holes
    ids[mask == 0] = 0
    mi = np.zeros((B, 2, 3), np.int32)
    mm = np.zeros((B, 2, 3), np.float32)
    for b in range(B):
        n = max(int(lengths[b]), 4)
        mi[b] = r.integers(0, n, size=(2, 3))
        mm[b] = 1
    mi[2, 1, 2] = L - 7  # a marker past the row's last unmasked token
    mi[1, 0, 1], mm[1, 0, 1] = L - 1, 0  # masked slot: does not extend the row
    mm[5, 1] = 0
    return ids, mask, mi, mm


def _small_pair(seed=13, **flags):
    from gliner_decide import GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    w = synthetic_weights(pc, seed=seed)
    return GLiNERDecideClassifier(w, pc, **flags), GLiNERDecideClassifier(w, pc, full_rows=True), w, pc


def test_compact_last_layer_edges():
    """The last layer on the marker rows only: a row whose marker slots are
    all masked (no query computed; its logits are all -10000) and more marker
    slots than tokens (B*Hh*O = 240 > B*L = 128, after a larger batch grew the
    workspace).  Padded and packed, the logits equal GD_FULL_ROWS bit for
    bit."""
    from gliner_decide import DecisionInput
    fast, full, _, _ = _small_pair(seed=23)
    big = _extent_batch(128, 5)
    fast.classify(DecisionInput(*big))  # workspace for 768 tokens
    r = np.random.default_rng(31)
    B, L, Hh, O = 4, 32, 3, 20
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    lengths = np.array([32, 20, 9, 25])
    mask = (np.arange(L)[None] < lengths[:, None]).astype(np.float16)
    ids[mask == 0] = 0
    mi = r.integers(0, L, size=(B, Hh, O)).astype(np.int32)
    mm = (r.random((B, Hh, O)) < 0.7).astype(np.float32)
    mm[2] = 0  # every slot of row 2 masked
    inp = DecisionInput(ids, mask, mi, mm)
    want = full.classify_device(*inp.to_device()).float().cpu().numpy()
    assert np.all(want[2] == -10000.0)
    padded = fast.classify_device(*inp.to_device()).float().cpu().numpy()
    packed = fast.classify(inp).logits.float().cpu().numpy()
    np.testing.assert_array_equal(padded, want)
    np.testing.assert_array_equal(packed, want)
    fast.check_device_errors()


def test_compact_last_layer_on_skinny_tiles():
    """Ten marker rows: the last layer's products after the attention run on
    the 32 x 16 skinny tiles (at most 32 rows), while GD_FULL_ROWS runs them
    on all 64 token rows with the 64 x 64 tiles.  The logits agree bit for
    bit: both kernels accumulate every element in the same order."""
    from gliner_decide import DecisionInput
    fast, full, _, _ = _small_pair(seed=29)
    r = np.random.default_rng(37)
    B, L, Hh, O = 2, 32, 1, 5
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    mask = np.ones((B, L), np.float16)
    mi = r.integers(0, L, size=(B, Hh, O)).astype(np.int32)
    mm = np.ones((B, Hh, O), np.float32)
    inp = DecisionInput(ids, mask, mi, mm)
    want = full.classify_device(*inp.to_device()).float().cpu().numpy()
    got = fast.classify_device(*inp.to_device()).float().cpu().numpy()
    assert np.all(np.isfinite(want))
    np.testing.assert_array_equal(got, want)
    fast.check_device_errors()


@pytest.mark.parametrize("L", [128, 256, 512])
def test_row_extents_leave_logits_unchanged(L):
    """classify stops each row's attention at its extent (last unmasked or
    marker-read position + 1); the logits must equal those of the full
    computation (GD_FULL_ROWS) bit for bit.  The packed forward (only the
    extents' tokens through every kernel) must agree within fp16 rounding of
    the differently tiled small GEMMs."""
    from gliner_decide import DecisionInput
    fast, full, _, _ = _small_pair()
    ids, mask, mi, mm = _extent_batch(L, L)
    inp = DecisionInput(ids, mask, mi, mm)
    dev = inp.to_device()
    a = fast.classify_device(*dev).float().cpu().numpy()
    b_ = full.classify_device(*dev).float().cpu().numpy()
    assert np.all(np.isfinite(a)) and np.all(a[mm == 0] == -10000.0)
    np.testing.assert_array_equal(a, b_)
    packed = fast.classify(inp).logits.float().cpu().numpy()  # host arrays: packed rows
    assert np.all(packed[mm == 0] == -10000.0)
    assert np.max(np.abs(packed - a)) <= 2e-3


def test_packed_rows_match_padded_at_full_size():
    """B=32, L=256, lengths U[40, 256] (the classification workload's
    layout): packed rows (4.9k of 8.2k tokens) give the padded forward's
    logits bit for bit (both run the 256-row MFMA GEMM tiles), eagerly and
    through a captured graph; a wrong token total raises the device flag."""
    from gliner_decide import DecisionInput
    from gliner_decide._native import GlinerDecideError
    from gliner_decide.decode import row_extents
    from gliner_decide.synthetic import classification_batch
    fast, full, w, pc = _small_pair(seed=17)
    batch = classification_batch(seed=4, vocab=3000)
    a = batch.arrays()
    a["input_ids"] = np.where(a["input_ids"] >= 3000, a["input_ids"] % 3000, a["input_ids"])  # marker ids
    total = int(row_extents(a["attention_mask"], a["marker_indices"], a["marker_mask"]).sum())
    assert 2048 < total < 8192
    dev = DecisionInput(**a).to_device()
    padded = fast.classify_device(*dev).float().cpu().numpy()
    packed = fast.classify_device(*dev, total_tokens=total).float().cpu().numpy()
    np.testing.assert_array_equal(packed, padded)
    from gliner_decide import GLiNERDecideClassifier
    graph = GLiNERDecideClassifier(w, pc, use_compiled_graph=True)
    for _ in range(3):
        g = graph.classify_device(*dev, total_tokens=total).float().cpu().numpy()
        np.testing.assert_array_equal(g, padded)
    # another batch whose total lands in the same 256-token capacity replays
    # that graph (graphs are keyed by capacity, not by total)
    a2 = {k: v.copy() for k, v in a.items()}
    lens = a2["attention_mask"].astype(np.float32).sum(1).astype(int)
    cut = min(9, (total - 1) % 256)
    b0 = int(np.argmax(lens))
    a2["attention_mask"][b0, lens[b0] - cut:] = 0
    total2 = int(row_extents(a2["attention_mask"], a2["marker_indices"], a2["marker_mask"]).sum())
    assert total2 == total - cut and (total2 + 255) // 256 == (total + 255) // 256
    dev2 = DecisionInput(**a2).to_device()
    eager2 = fast.classify_device(*dev2, total_tokens=total2).float().cpu().numpy()
    for _ in range(2):
        g2 = graph.classify_device(*dev2, total_tokens=total2).float().cpu().numpy()
        np.testing.assert_array_equal(g2, eager2)
    graph.check_device_errors()
    fast.check_device_errors()
    fast.classify_device(*dev, total_tokens=total - 1)
    with pytest.raises(GlinerDecideError):
        fast.check_device_errors()
    fast.check_device_errors()  # cleared
    with pytest.raises(GlinerDecideError):
        fast.classify_device(*dev, total_tokens=8192 + 1)


def test_compiled_graph_replays_match_eager():
    from gliner_decide import DecisionInput, GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    w = synthetic_weights(pc, seed=3)
    eager = GLiNERDecideClassifier(w, pc)
    graph = GLiNERDecideClassifier(w, pc, use_compiled_graph=True)
    r = np.random.default_rng(4)
    for trial in range(4):
        B, L = (2, 32) if trial % 2 == 0 else (3, 96)
        ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
        mask = np.ones((B, L), np.float16)
        mask[-1, L // 2:] = 0
        mi = np.tile(np.arange(1, 6, dtype=np.int32), (B, 1, 1))
        mm = np.ones((B, 1, 5), np.float32)
        inp = DecisionInput(ids, mask, mi, mm)
        a = eager.classify(inp).logits.float().cpu().numpy()
        b = graph.classify(inp).logits.float().cpu().numpy()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(a, b)


def test_profile_events_and_same_logits():
    from gliner_decide import DecisionInput
    gpu, w, pc, oc = _models(dict(num_hidden_layers=2, vocab_size=3000), seed=5)
    r = np.random.default_rng(6)
    ids = r.integers(1000, 3000, size=(2, 32)).astype(np.int32)
    inp = DecisionInput(ids, np.ones((2, 32), np.float16), np.ones((2, 1, 3), np.int32), np.ones((2, 1, 3), np.float32))
    a = gpu.classify(inp).logits.float().cpu().numpy()
    res = gpu.classify(inp, collect_profile=True)
    names = [e.name for e in res.events]
    assert names[0] == "embedding" and names[-1] == "classifier"
    assert "layer_1_feed_forward" in names and len(names) == 2 + 4 * 2
    np.testing.assert_array_equal(res.logits.float().cpu().numpy(), a)


def test_device_index_errors_reported():
    from gliner_decide import DecisionInput, GlinerDecideError
    gpu, w, pc, oc = _models(dict(num_hidden_layers=1, vocab_size=3000), seed=5)
    ids = np.full((1, 32), 5000, np.int32)  # >= vocab
    inp = DecisionInput(ids, np.ones((1, 32), np.float16), np.ones((1, 1, 2), np.int32),
                        np.ones((1, 1, 2), np.float32))
    gpu.classify(inp)
    with pytest.raises(GlinerDecideError):
        gpu.check_device_errors()
    gpu.check_device_errors()  # cleared


def _probs_and_sets(logits, tasks):
    out = []
    for b in range(logits.shape[0]):
        out.append(O.decode(logits[b], tasks[b]))
    return out


def _margin(probs, multi):
    """Distance of a head's decision from a tie: |p - 0.5| nearest the
    threshold for multi-label heads, the top-two gap for single-label ones."""
    p = np.asarray(probs, np.float64)
    if multi:
        return float(np.min(np.abs(p - 0.5)))
    srt = np.sort(p)[::-1]
    return float(srt[0] - srt[1]) if len(srt) > 1 else 1.0


def compare_decisions(got_logits, want_logits, tasks, tol=1e-3):
    """Label probabilities within tol, and identical selected label sets
    (argmax for single-label heads, p >= 0.5 for multi-label heads) except
    where the GPU's and the reference's decisions both lie within 2 * tol of
    a tie: there two evaluations of the same fp16 rounding chain that differ
    by less than the tolerance fall on different sides.  Returns
    (near_ties, split): the count of heads within 2 * tol of a tie on the
    reference side, and the (row, head) pairs whose label sets differ."""
    g = _probs_and_sets(got_logits, tasks)
    w = _probs_and_sets(want_logits, tasks)
    near_ties, split = 0, []
    for b, (gr, wr) in enumerate(zip(g, w)):
        for h, ((gs, gp), (ws, wp)) in enumerate(zip(gr, wr)):
            assert np.max(np.abs(np.asarray(gp) - np.asarray(wp))) <= tol, (b, h)
            multi = tasks[b][h][1]
            m_want, m_got = _margin(wp, multi), _margin(gp, multi)
            near_ties += int(m_want <= 2 * tol)
            if gs != ws:
                assert m_want <= 2 * tol and m_got <= 2 * tol, (b, h, gs, ws, m_want, m_got)
                split.append((b, h))
    return near_ties, split


def _restated(w, oc, arrays, rows=None, chunk=16):
    """Logits of the batched torch fp32 restatement with the fp16 rounding
    points (oracle/torch_cpu.py, round16=True), in chunks of rows."""
    from oracle.torch_cpu import TorchCPUModel
    m = TorchCPUModel(w, oc, round16=True)
    keys = ("input_ids", "attention_mask", "marker_indices", "marker_mask")
    rows = np.arange(arrays["input_ids"].shape[0]) if rows is None else np.asarray(rows)
    out = [m.forward(*(arrays[k][rows[i:i + chunk]] for k in keys)).numpy() for i in range(0, len(rows), chunk)]
    return np.concatenate(out)


def _oracle_rows(om, arrays, rows):
    return om.forward(*(arrays[k][rows] for k in ("input_ids", "attention_mask", "marker_indices", "marker_mask")))


def _full_model(seed):
    gpu, w, pc, oc = _models(dict(vocab_size=128100), seed=seed)
    return gpu, w, oc


@pytest.fixture(scope="module")
def classify_run():
    """The 24-layer encoder + classifier at B=32, L=256 (lengths U[40, 256],
    one task of 5 labels), through the GPU once."""
    from gliner_decide import DecisionInput
    from gliner_decide.synthetic import classification_batch
    gpu, w, oc = _full_model(4)
    batch = classification_batch(seed=4)
    got = gpu.classify(DecisionInput(**batch.arrays())).logits.float().cpu().numpy()
    return dict(w=w, oc=oc, batch=batch, a=batch.arrays(), got=got)


def test_full_model_classify_workload(classify_run):
    """Every row against the fp16-rounding torch restatement at the decision
    bar (probabilities within 1e-3, identical argmax), and against the
    restatement without fp16 rounding points: logits within 5e-3 (the fp16
    chain's own distance from exact arithmetic, 2.1e-3 measured)."""
    from oracle.torch_cpu import TorchCPUModel
    d = classify_run
    got, a, batch = d["got"], d["a"], d["batch"]
    assert got.shape == (32, 1, 5) and np.all(np.isfinite(got))
    near, split = compare_decisions(got, _restated(d["w"], d["oc"], a), batch.tasks)
    d["split"] = sorted({b for b, _ in split})
    print(f"B=32 L=256: 32 rows against the rounding restatement, {near} heads within 2e-3 of a tie, "
          f"label sets split on {split}")
    assert len(split) <= max(1, near // 4)
    exact = TorchCPUModel(d["w"], d["oc"]).forward(a["input_ids"], a["attention_mask"], a["marker_indices"],
                                                    a["marker_mask"]).numpy()
    assert np.max(np.abs(got - exact)) <= 5e-3, np.max(np.abs(got - exact))


def test_full_model_classify_oracle_rows(classify_run):
    """The float64 oracle (fp16 rounding points) recomputes 5 rows -- the
    shortest, the longest and three others; rows are independent -- plus any
    row whose label set split against the torch restatement, at the
    decision bar."""
    d = classify_run
    a = d["a"]
    om = O.OracleModel(O.ModelWeights.from_store(d["w"], d["oc"]), d["oc"], dtype=np.float64)
    lens = (a["attention_mask"] > 0).sum(1)
    rows = sorted({int(np.argmin(lens)), int(np.argmax(lens)), 0, 17, 25} | set(d.get("split", [])))
    near, split = compare_decisions(d["got"][rows], _oracle_rows(om, a, rows), [d["batch"].tasks[i] for i in rows])
    print(f"B=32 L=256: oracle rows {rows}, {near} heads within 2e-3 of a tie, label sets split on "
          f"{[(rows[b], h) for b, h in split]}")


@pytest.fixture(scope="module")
def long_context_run():
    """B=64, L=512 (every row full), 3 task heads x 20 options (two
    multi-label heads of 20 labels, one single-label head of 8), through the
    GPU once."""
    from gliner_decide import DecisionInput
    from gliner_decide.synthetic import long_context_batch
    gpu, w, oc = _full_model(6)
    batch = long_context_batch(seed=6)
    a = batch.arrays()
    got = gpu.classify(DecisionInput(**a)).logits.float().cpu().numpy()
    return dict(w=w, oc=oc, batch=batch, a=a, got=got)


def _long_context_oracle_rows(a):
    """The rows whose schemas (last marker position) are shortest, median and
    longest, and the last row."""
    last = a["marker_indices"].reshape(a["marker_indices"].shape[0], -1).max(1)
    order = np.argsort(last, kind="stable")
    return sorted({int(order[0]), int(order[len(order) // 2]), int(order[-1]), len(order) - 1})


def test_long_context_workload(long_context_run):
    """Options past a head's label count read -10000; every row's three heads
    against the fp16-rounding torch restatement at the decision bar
    (probabilities within 1e-3, identical thresholded label sets and argmax)."""
    d = long_context_run
    got, a, batch = d["got"], d["a"], d["batch"]
    assert got.shape == (64, 3, 20) and np.all(np.isfinite(got))
    assert np.all(got[a["marker_mask"] == 0] == -10000.0)
    near, split = compare_decisions(got, _restated(d["w"], d["oc"], a, chunk=8), batch.tasks)
    d["split"] = sorted({b for b, _ in split})
    print(f"B=64 L=512: 64 rows x 3 heads against the rounding restatement, {near} heads within 2e-3 of a tie, "
          f"label sets split on {split}")
    assert len(split) <= max(1, near // 4)


@pytest.mark.parametrize("pick", [0, 1, 2, 3])
def test_long_context_oracle_rows(long_context_run, pick):
    """The float64 oracle recomputes 4 rows (shortest, median and longest
    schema, and the last row), all three heads each, at the decision bar."""
    d = long_context_run
    rows = _long_context_oracle_rows(d["a"])
    if pick >= len(rows):
        pytest.skip("fewer distinct rows")
    row = [rows[pick]]
    om = O.OracleModel(O.ModelWeights.from_store(d["w"], d["oc"]), d["oc"], dtype=np.float64)
    near, split = compare_decisions(d["got"][row], _oracle_rows(om, d["a"], row), [d["batch"].tasks[i] for i in row])
    print(f"B=64 L=512: oracle row {row[0]}, {near} heads within 2e-3 of a tie, label sets split on heads "
          f"{[h for _, h in split]}")


def test_long_context_split_rows_vs_oracle(long_context_run):
    """Rows whose label sets split against the torch restatement (near
    ties) are recomputed by the float64 oracle, at the decision bar."""
    d = long_context_run
    rows = [r for r in d.get("split", []) if r not in _long_context_oracle_rows(d["a"])]
    if not rows:
        pytest.skip("no row split against the torch restatement")
    om = O.OracleModel(O.ModelWeights.from_store(d["w"], d["oc"]), d["oc"], dtype=np.float64)
    near, split = compare_decisions(d["got"][rows], _oracle_rows(om, d["a"], rows), [d["batch"].tasks[i] for i in rows])
    print(f"B=64 L=512: oracle rows {rows}, {near} heads within 2e-3 of a tie, label sets split on "
          f"{[(rows[b], h) for b, h in split]}")


@pytest.fixture(scope="module")
def bucket_mix_run():
    """All 4096 rows of the mixed workload (buckets L = 32 ... 512, 1-2 tasks
    x 2-10 labels, B=32 with the last batch of a bucket padded by copies of
    its last valid row), through the GPU once."""
    from gliner_decide import DecisionInput
    from gliner_decide.synthetic import bucket_mix
    gpu, w, oc = _full_model(5)
    runs = []
    for x in bucket_mix(seed=5):
        runs.append((x, gpu.classify(DecisionInput(**x.arrays())).logits.float().cpu().numpy()))
    return dict(w=w, oc=oc, runs=runs)


def test_bucket_mix_workload(bucket_mix_run):
    """Every row runs; padded rows reproduce their source row's logits bit
    for bit."""
    rows_run, buckets = 0, set()
    for x, got in bucket_mix_run["runs"]:
        assert np.all(np.isfinite(got))
        v = x.valid_rows
        rows_run += v
        buckets.add(x.shape[1])
        if v < got.shape[0]:
            np.testing.assert_array_equal(got[v:], np.broadcast_to(got[v - 1], got[v:].shape))
    assert rows_run == 4096 and buckets == {32, 64, 96, 128, 256, 512}


def test_bucket_mix_batches_vs_restatement(bucket_mix_run):
    """One whole batch per bucket (each bucket's first) against the
    fp16-rounding torch restatement at the decision bar."""
    d = bucket_mix_run
    seen, near, split = set(), 0, []
    for x, got in d["runs"]:
        L = x.shape[1]
        if L in seen:
            continue
        seen.add(L)
        v = x.valid_rows
        a = {k: arr[:v] for k, arr in x.arrays().items()}
        n, sp = compare_decisions(got[:v], _restated(d["w"], d["oc"], a), x.tasks[:v])
        near += n
        split += [(L, b, h) for b, h in sp]
    assert seen == {32, 64, 96, 128, 256, 512}
    print(f"bucket mix: one batch per bucket against the rounding restatement, {near} heads within 2e-3 of a "
          f"tie, label sets split on (L, row, head) {split}")
    assert len(split) <= max(1, near // 4)


def test_bucket_mix_oracle_rows(bucket_mix_run):
    """The float64 oracle recomputes the last valid row of one batch per
    bucket at the decision bar."""
    d = bucket_mix_run
    om = O.OracleModel(O.ModelWeights.from_store(d["w"], d["oc"]), d["oc"], dtype=np.float64)
    checked = set()
    for x, got in d["runs"]:
        L = x.shape[1]
        if L not in checked:
            checked.add(L)
            rows = [x.valid_rows - 1]
            _, split = compare_decisions(got[rows], _oracle_rows(om, x.arrays(), rows), [x.tasks[i] for i in rows])
            assert not split, (L, split)
    assert checked == {32, 64, 96, 128, 256, 512}


# ---------------------------------------------------------------------------
# every constructor flag of GLiNERDecideClassifier.init (DeBERTa.swift:188-196)
# ---------------------------------------------------------------------------
FLAG_SETS = {
    "default": dict(),
    "fused_kernels": dict(use_fused_kernels=True),
    "generic_attention": dict(use_fast_attention=False),
    "custom_relative_kernel": dict(use_custom_relative_kernel=True),
    "custom_relative_generic": dict(use_custom_relative_kernel=True, use_fast_attention=False),
    "fused_attention_kernel": dict(use_fused_attention_kernel=True),
}


@pytest.mark.parametrize("name", sorted(FLAG_SETS))
def test_classifier_flags_match_oracle(name):
    """Two full-width layers + head with padded rows under each flag set,
    against OracleModel with the same flags: hidden states and logits, with
    the bar of the default-path test (the spread between the float64 and
    float32 restatements, x2, floor 2e-3).  Packed, padded and full-row
    classify agree bit for bit.  Row 3 has no valid token but unmasked
    marker slots: the reference's degenerate softmax over every key
    (DeBERTa.swift:329-335 with an all-zero mask) reaches its logits."""
    from gliner_decide import DecisionInput, GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    flags = FLAG_SETS[name]
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    w = synthetic_weights(pc, seed=19)
    oc = O.Config(**{k: getattr(pc, k) for k in O.Config.__dataclass_fields__})
    gpu = GLiNERDecideClassifier(w, pc, **flags)
    full = GLiNERDecideClassifier(w, pc, full_rows=True, **flags)
    r = np.random.default_rng(5)
    B, L = 4, 96
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    lengths = np.array([96, 61, 17, 0])
    mask = (np.arange(L)[None] < lengths[:, None]).astype(np.float16)
    ids[mask == 0] = 0
    mi = np.array([[[1, 2, 3, 4], [5, 6, 0, 0]]] * B, np.int32)
    mm = np.array([[[1, 1, 1, 1], [1, 1, 0, 0]]] * B, np.float32)
    inp = DecisionInput(ids, mask, mi, mm)
    packed = gpu.classify(inp).logits.float().cpu().numpy()
    padded = gpu.classify_device(*inp.to_device()).float().cpu().numpy()
    every = full.classify_device(*inp.to_device()).float().cpu().numpy()
    np.testing.assert_array_equal(packed, every)
    np.testing.assert_array_equal(padded, every)
    hid = gpu.encode(inp).float().cpu().numpy()
    mw = O.ModelWeights.from_store(w, oc)
    om = O.OracleModel(mw, oc, **flags)
    want_h = om.encode(ids, mask)
    om32 = O.OracleModel(O.ModelWeights.from_store(w, oc), oc, dtype=np.float32, **flags)
    floor = np.max(np.abs(om32.encode(ids, mask).astype(np.float64) - want_h))
    err = np.max(np.abs(hid - want_h))
    assert err <= max(2e-3, 2 * floor), (name, err, floor)
    want_logits = O.classifier_head(want_h, mi, mm, mw)
    assert np.all(packed[mm == 0] == -10000.0)
    assert np.max(np.abs(packed - want_logits)) <= 2e-3, name
    # and the flag changes the computation: the default graph's logits differ
    if name not in ("default", "fused_kernels"):
        base = GLiNERDecideClassifier(w, pc).classify(inp).logits.float().cpu().numpy()
        assert not np.array_equal(base, packed), name


def test_safetensors_checkpoint_matches_oracle(tmp_path):
    """The path of WeightStore(url:) (Weights.swift:26-28) over the format of
    prepare_model.py:82-113: weights written with safetensors, read by the
    library's own parser (gd_weight_store_load_safetensors), then classify.
    The logits equal those of the classifier built from the same arrays
    through gd_weight_store_add (bit for bit), and the oracle built from the
    file's arrays (read back by the safetensors package) within 2e-3."""
    from safetensors.numpy import load_file, save_file
    from gliner_decide import DecisionInput, GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    from gliner_decide.weights import WeightStore
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    w = synthetic_weights(pc, seed=29)
    path = tmp_path / "gliner_decide_fp16.safetensors"
    save_file(w, str(path), metadata={"precision": "float16", "scope": "encoder+classification-only"})
    store = WeightStore(url=path)
    assert len(store) == len(w)
    from_file = GLiNERDecideClassifier(store, pc)
    from_arrays = GLiNERDecideClassifier(w, pc)
    r = np.random.default_rng(3)
    B, L = 2, 64
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    mask = (np.arange(L)[None] < np.array([[64], [33]])).astype(np.float16)
    ids[mask == 0] = 0
    mi = np.array([[[1, 2, 3]]] * B, np.int32)
    mm = np.ones((B, 1, 3), np.float32)
    inp = DecisionInput(ids, mask, mi, mm)
    got = from_file.classify(inp).logits.float().cpu().numpy()
    np.testing.assert_array_equal(got, from_arrays.classify(inp).logits.float().cpu().numpy())
    oc = O.Config(**{k: getattr(pc, k) for k in O.Config.__dataclass_fields__})
    om = O.OracleModel(O.ModelWeights.from_store(load_file(str(path)), oc), oc)
    assert np.max(np.abs(got - om.forward(ids, mask, mi, mm))) <= 2e-3
