"""The classify that allocates nothing (gd_classifier_classify_static):
through the C-ABI, its logits equal those of gd_classifier_classify_packed
and gd_classifier_classify on the same inputs, bit for bit, on two calls in a
row (the second smaller), without the context growing its device memory;
calls beyond the static workspace are refused with GD_ERR_SHAPE.  Calls on
two streams with no synchronisation between them are ordered by the per-GPU
event, and the call captured into a graph replays bit-exactly."""

import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _batch(r, B, L, lengths):
    ids = r.integers(1000, 3000, size=(B, L)).astype(np.int32)
    mask = (np.arange(L)[None] < np.asarray(lengths)[:, None]).astype(np.float16)
    ids[mask == 0] = 0
    mi = np.stack([r.integers(0, max(int(n), 1), size=(2, 3)) for n in lengths]).astype(np.int32)
    mm = (r.random((B, 2, 3)) < 0.8).astype(np.float32)
    return ids, mask, mi, mm


def _call(fn, model, arrays, total):
    from gliner_decide import _native as N
    from gliner_decide import DecisionInput
    from gliner_decide.device import stream_handle
    ids, mask, mi, mm = DecisionInput(*arrays).to_device()
    B, L = ids.shape
    _, Hh, O = mi.shape
    out = torch.full((B, Hh, O), float("nan"), dtype=torch.float16, device=ids.device)
    args = [model._h, ids.data_ptr(), mask.data_ptr(), mi.data_ptr(), mm.data_ptr(), B, L, Hh, O]
    if total is not None:
        args.append(total)
    status = getattr(N.lib(), fn)(*args, out.data_ptr(), stream_handle())
    torch.cuda.synchronize()
    return status, out.cpu().numpy().view(np.uint16)


def test_static_classify_matches_allocating_entry_points():
    from gliner_decide import GLiNERDecideClassifier
    from gliner_decide import _native as N
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.decode import row_extents
    from gliner_decide.synthetic import synthetic_weights
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    w = synthetic_weights(pc, seed=37)
    quiet = GLiNERDecideClassifier(w, pc)  # only ever called through the static entry point
    ref = GLiNERDecideClassifier(w, pc)
    bytes0 = quiet.device_bytes
    r = np.random.default_rng(41)
    for B, L, lengths in ((4, 256, [256, 200, 97, 33]), (2, 64, [64, 17])):
        arrays = _batch(r, B, L, lengths)
        total = int(row_extents(arrays[1], arrays[2], arrays[3]).sum())
        st, packed_static = _call("gd_classifier_classify_static", quiet, arrays, total)
        assert st == N.GD_OK, N.last_error()
        st, padded_static = _call("gd_classifier_classify_static", quiet, arrays, -1)
        assert st == N.GD_OK, N.last_error()
        st, packed = _call("gd_classifier_classify_packed", ref, arrays, total)
        assert st == N.GD_OK
        st, padded = _call("gd_classifier_classify", ref, arrays, None)
        assert st == N.GD_OK
        np.testing.assert_array_equal(packed_static, packed)
        np.testing.assert_array_equal(padded_static, padded)
        np.testing.assert_array_equal(padded_static, packed)
        assert quiet.device_bytes == bytes0  # the context allocated nothing
    quiet.check_device_errors()
    # beyond the static workspace: 16 x 256 padded tokens (the packed total of
    # the same rows fits)
    arrays = _batch(r, 16, 256, [100] * 16)
    st, _ = _call("gd_classifier_classify_static", quiet, arrays, -1)
    assert st == N.GD_ERR_SHAPE and "static workspace" in N.last_error()
    total = int(row_extents(arrays[1], arrays[2], arrays[3]).sum())
    assert total <= 2048
    st, got = _call("gd_classifier_classify_static", quiet, arrays, total)
    assert st == N.GD_OK
    st, want = _call("gd_classifier_classify_packed", ref, arrays, total)
    np.testing.assert_array_equal(got, want)
    assert quiet.device_bytes == bytes0


def _device_inputs(arrays):
    from gliner_decide import DecisionInput
    return list(DecisionInput(*arrays).to_device())


def _static(model, dev, total, out, stream):
    from gliner_decide import _native as N
    ids, mask, mi, mm = dev
    B, L = ids.shape
    _, Hh, O = mi.shape
    return N.lib().gd_classifier_classify_static(model._h, ids.data_ptr(), mask.data_ptr(), mi.data_ptr(),
                                                 mm.data_ptr(), B, L, Hh, O, total, out.data_ptr(), stream)


def _two_layer_models(seed):
    from gliner_decide import GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    pc = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    w = synthetic_weights(pc, seed=seed)
    return GLiNERDecideClassifier(w, pc), GLiNERDecideClassifier(w, pc)


def test_static_calls_on_two_streams_are_ordered():
    """Two calls on two streams with no synchronisation between them share
    the GPU's static workspace; the per-GPU event runs them one after the
    other, so each returns its own inputs' logits."""
    from gliner_decide import _native as N
    from gliner_decide.decode import row_extents
    quiet, ref = _two_layer_models(53)
    r = np.random.default_rng(59)
    sets = [_batch(r, 4, 256, [256, 190, 120, 40]), _batch(r, 4, 256, [64, 250, 256, 129])]
    want = [_call("gd_classifier_classify", ref, a, None)[1] for a in sets]
    totals = [int(row_extents(a[1], a[2], a[3]).sum()) for a in sets]
    for total_mode in ("padded", "packed"):
        devs = [_device_inputs(a) for a in sets]
        outs = [torch.full((4, 2, 3), float("nan"), dtype=torch.float16, device="cuda") for _ in sets]
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        torch.cuda.synchronize()
        for i in range(2):
            total = -1 if total_mode == "padded" else totals[i]
            assert _static(quiet, devs[i], total, outs[i], streams[i].cuda_stream) == N.GD_OK, N.last_error()
        torch.cuda.synchronize()
        for i in range(2):
            np.testing.assert_array_equal(outs[i].cpu().numpy().view(np.uint16), want[i])


def test_static_classify_captured_graph_replays():
    """classify_static captured into a graph (one eager call first) and
    replayed several times, with new inputs copied into the captured buffers,
    other static calls and synchronisations between the replays: every
    replay equals the allocating entry point's logits bit for bit."""
    from gliner_decide import _native as N
    from gliner_decide.decode import row_extents
    quiet, ref = _two_layer_models(61)
    r = np.random.default_rng(67)
    base = _batch(r, 4, 256, [256, 170, 90, 33])
    # same extents and markers, other token ids: the packed total is unchanged
    other_ids = r.integers(1000, 3000, size=base[0].shape).astype(np.int32)
    other_ids[base[1] == 0] = 0
    variants = [base, (other_ids,) + tuple(base[1:])]
    total = int(row_extents(base[1], base[2], base[3]).sum())
    distractor = _device_inputs(_batch(r, 2, 128, [128, 77]))
    scratch_out = torch.empty((2, 2, 3), dtype=torch.float16, device="cuda")
    for mode_total in (-1, total):
        dev = _device_inputs(base)
        out = torch.full((4, 2, 3), float("nan"), dtype=torch.float16, device="cuda")
        assert _static(quiet, dev, mode_total, out, torch.cuda.current_stream().cuda_stream) == N.GD_OK
        torch.cuda.synchronize()
        eager = out.cpu().numpy().view(np.uint16).copy()
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        with torch.cuda.graph(g, stream=side):
            st = _static(quiet, dev, mode_total, out, torch.cuda.current_stream().cuda_stream)
        assert st == N.GD_OK, N.last_error()
        for rep, v in enumerate([0, 1, 0, 1, 1]):
            want = _call("gd_classifier_classify" if mode_total < 0 else "gd_classifier_classify_packed", ref,
                         variants[v], None if mode_total < 0 else total)[1]
            if v == 0:
                np.testing.assert_array_equal(want, eager)
            for t, src in zip(dev, _device_inputs(variants[v])):
                t.copy_(src)
            out.fill_(float("nan"))
            # eager work on the same static workspace between replays
            assert _static(quiet, distractor, -1, scratch_out, torch.cuda.current_stream().cuda_stream) == N.GD_OK
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), want, err_msg=f"replay {rep}")
        del g
    quiet.check_device_errors()

