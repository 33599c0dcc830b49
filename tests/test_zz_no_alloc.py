"""The classify that allocates nothing (gd_classifier_classify_static):
through the C-ABI, its logits equal those of gd_classifier_classify_packed
and gd_classifier_classify on the same inputs, bit for bit, on two calls in a
row (the second smaller), without the context growing its device memory;
calls beyond the static workspace are refused with GD_ERR_SHAPE."""

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
