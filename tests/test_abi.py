"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/gliner_decide.h declares, and rejects bad arguments and bad weights
with status codes (the reference traps on `precondition` instead) before any
device work.  No kernel is launched here."""

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from gliner_decide import _native as N

HEADERS = [Path(__file__).resolve().parents[1] / "include" / h for h in ("gliner_decide.h", "gliner_decide_diag.h")]


def declared_functions():
    text = "\n".join(h.read_text() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|void|char\s*\*|int64_t|char)\s*\**\s*(gd_\w+)\s*\(",
                                 text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(N.EXPORTED_SYMBOLS)
    assert lib.gd_abi_version() == 1
    assert b"gfx950" in lib.gd_build_info()


def test_config_default_matches_reference():
    c = N.GdConfig()
    N.lib().gd_config_default(C.byref(c))
    assert (c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads) == (1024, 4096, 24, 16)
    assert abs(c.layer_norm_eps - 1e-7) < 1e-12 and c.position_buckets == 256 and c.max_relative_positions == -1
    assert c.vocab_size == 128011 and c.classifier_hidden == 2048 and c.pad_token_id == 0


FAKE = 0x10000  # never dereferenced: validation fails before any launch


def test_argument_validation_without_device():
    lib = N.lib()
    assert lib.gd_residual_layer_norm(None, None, None, None, None, 4, 1024, 1e-7, 0, None) == N.GD_ERR_INVALID_ARGUMENT
    assert "null" in N.last_error()
    assert lib.gd_residual_layer_norm(FAKE, None, FAKE, FAKE, FAKE, 4, 1020, 1e-7, 0, None) == N.GD_ERR_SHAPE
    assert lib.gd_residual_layer_norm(FAKE, None, FAKE, FAKE, FAKE, 4, 1024, 0.0, 0, None) == N.GD_ERR_INVALID_ARGUMENT
    assert lib.gd_residual_layer_norm(FAKE, None, FAKE, FAKE, FAKE, 4, 1024, 1e-7, 8, None) == N.GD_ERR_INVALID_ARGUMENT
    assert lib.gd_linear(FAKE, FAKE, FAKE, FAKE, 8, 100, 64, 64, 100, None, 0, 1, None) == N.GD_ERR_SHAPE
    assert lib.gd_linear(FAKE, FAKE, FAKE, FAKE, 8, 128, 60, 64, 128, None, 0, 1, None) == N.GD_ERR_SHAPE
    assert lib.gd_linear(FAKE, FAKE, None, FAKE, 8, 128, 64, 64, 128, None, 0, 1, None) == N.GD_ERR_INVALID_ARGUMENT
    assert lib.gd_linear(FAKE, FAKE, FAKE, FAKE, 8, 128, 64, 64, 128, FAKE, 0, 1, None) == N.GD_ERR_SHAPE
    assert lib.gd_linear(FAKE, FAKE, FAKE, FAKE, 8, 128, 64, 64, 128, None, 0, 9, None) == N.GD_ERR_INVALID_ARGUMENT
    # the tile kernels store C in 16-byte row segments
    assert lib.gd_linear(FAKE, FAKE, FAKE, FAKE + 8, 8, 128, 64, 64, 128, None, 0, 1, None) == N.GD_ERR_INVALID_ARGUMENT
    assert "16-byte" in N.last_error()
    bh = N.GdBhld(FAKE, 0, 0, 64)
    tb = N.GdTable(FAKE, 512 * 64, 64)
    assert lib.gd_deberta_attention(bh, bh, bh, tb, tb, FAKE, 0, 1, 1, 40, 64, 512, 256, 0, FAKE, 40, None) == \
        N.GD_ERR_SHAPE  # L = 40 is not a multiple of 16
    assert lib.gd_deberta_attention(bh, bh, bh, tb, tb, FAKE, 0, 1, 1, 64, 32, 512, 256, 0, FAKE, 64, None) == \
        N.GD_ERR_SHAPE  # head_dim 32
    assert lib.gd_deberta_attention(bh, bh, bh, tb, tb, FAKE, 0, 1, 1, 1024, 64, 512, 256, 0, FAKE, 64, None) == \
        N.GD_ERR_SHAPE  # L > 512
    assert lib.gd_deberta_attention(bh, bh, bh, tb, tb, FAKE, 3, 1, 1, 64, 64, 512, 256, 0, FAKE, 64, None) == \
        N.GD_ERR_INVALID_ARGUMENT  # mask kind
    assert lib.gd_relative_index_table(FAKE, 600, 256, 512, None) == N.GD_ERR_SHAPE


def _store_with(arrays):
    from gliner_decide.weights import WeightStore
    return WeightStore(arrays=arrays)


def _tiny_weights(**drop):
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights
    cfg = DeBERTaV2Configuration(hidden_size=128, intermediate_size=256, num_hidden_layers=1, num_attention_heads=2,
                                 vocab_size=64, classifier_hidden=128)
    return cfg, synthetic_weights(cfg, seed=0)


def _create(cfg, weights):
    store = _store_with(weights)
    h = C.c_void_p()
    c = cfg.to_native()
    st = N.lib().gd_classifier_create(C.byref(h), store.handle, C.byref(c), 0, None)
    if st == N.GD_OK:  # pragma: no cover - only on a GPU host
        N.lib().gd_classifier_destroy(h)
    return st


def test_weight_checks_before_device():
    cfg, w = _tiny_weights()
    missing = dict(w)
    del missing["encoder.encoder.layer.0.output.dense.bias"]
    assert _create(cfg, missing) == N.GD_ERR_MISSING_WEIGHT
    assert "Missing model weight: encoder.encoder.layer.0.output.dense.bias" in N.last_error()
    bad = dict(w)
    bad["encoder.encoder.rel_embeddings.weight"] = np.zeros((256, 128), np.float16)
    assert _create(cfg, bad) == N.GD_ERR_WEIGHT_SHAPE
    assert "expected [512, 128]" in N.last_error()
    f32 = dict(w)
    f32["classifier.0.bias"] = f32["classifier.0.bias"].astype(np.float32)
    assert _create(cfg, f32) == N.GD_ERR_WEIGHT_DTYPE
    from gliner_decide.config import DeBERTaV2Configuration
    bad_cfg = DeBERTaV2Configuration(hidden_size=128, num_attention_heads=4, intermediate_size=256,
                                     num_hidden_layers=1, vocab_size=64, classifier_hidden=128)  # head size 32
    assert _create(bad_cfg, w) == N.GD_ERR_INVALID_ARGUMENT


def test_safetensors_roundtrip(tmp_path):
    from safetensors.numpy import save_file
    from gliner_decide.weights import WeightStore
    _, w = _tiny_weights()
    path = tmp_path / "w.safetensors"
    save_file(w, str(path), metadata={"precision": "float16", "scope": "encoder+classification-only"})
    store = WeightStore(url=path)
    assert len(store) == len(w)
    # every tensor reads back with its shape, dtype and bytes (a wrong data
    # offset, header base or dtype mapping would show here)
    for key, arr in w.items():
        got = store.array(key)
        assert got.dtype == arr.dtype and got.shape == arr.shape, key
        np.testing.assert_array_equal(got.view(np.uint16), arr.view(np.uint16), err_msg=key)
    # mixed dtypes and ranks: offsets of later tensors depend on the sizes of earlier ones
    mixed = {"a": np.arange(6, dtype=np.float32).reshape(2, 3), "b": np.array([7, -9], np.int64),
             "c": np.arange(5, dtype=np.int32), "d": np.float16(1.5) * np.ones((3, 1, 2), np.float16),
             "s": np.array(3.25, np.float32)}
    save_file(mixed, str(tmp_path / "m.safetensors"))
    ms = WeightStore(url=tmp_path / "m.safetensors")
    for key, arr in mixed.items():
        got = ms.array(key)
        assert got.dtype == arr.dtype and got.shape == arr.shape, key
        np.testing.assert_array_equal(got, arr)
    with pytest.raises(N.GlinerDecideError) as e:
        ms.array("missing")
    assert e.value.status == N.GD_ERR_MISSING_WEIGHT
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{not json")
    with pytest.raises(N.GlinerDecideError) as e:
        WeightStore(url=bad)
    assert e.value.status == N.GD_ERR_IO
    with pytest.raises(N.GlinerDecideError):
        WeightStore(url=tmp_path / "nope.safetensors")


def _raw_safetensors(path, header: bytes, payload: bytes = b"\0" * 16):
    import struct
    path.write_bytes(struct.pack("<Q", len(header)) + header + payload)
    return path


@pytest.mark.parametrize("header", [
    # negative dimension with end < begin: both sides of the size check are -2
    b'{"x": {"dtype": "F16", "shape": [-1], "data_offsets": [2, 0]}}',
    # an integer beyond int64
    b'{"x": {"dtype": "F16", "shape": [99999999999999999999999], "data_offsets": [0, 2]}}',
    # a size that overflows int64 while every dimension fits
    b'{"x": {"dtype": "F16", "shape": [4294967296, 4294967296], "data_offsets": [0, 0]}}',
    # a range past the end of the file
    b'{"x": {"dtype": "F16", "shape": [64], "data_offsets": [0, 128]}}',
    # end before begin with a matching (negative) size is still rejected
    b'{"x": {"dtype": "F16", "shape": [], "data_offsets": [4, 2]}}',
])
def test_safetensors_malformed_headers_return_io_error(tmp_path, header):
    """Crafted headers are rejected with GD_ERR_IO; the process survives."""
    from gliner_decide.weights import WeightStore
    with pytest.raises(N.GlinerDecideError) as e:
        WeightStore(url=_raw_safetensors(tmp_path / "h.safetensors", header))
    assert e.value.status == N.GD_ERR_IO


def test_weight_store_add_rejects_overflowing_shape():
    from gliner_decide.weights import WeightStore
    import ctypes as C
    store = WeightStore()
    shape = (C.c_int64 * 2)(1 << 40, 1 << 40)
    buf = np.zeros(4, np.float16)
    assert N.lib().gd_weight_store_add(store.handle, b"x", buf.ctypes.data_as(C.c_void_p), N.GD_F16, shape, 2) \
        == N.GD_ERR_INVALID_ARGUMENT
    shape = (C.c_int64 * 1)(-3)
    assert N.lib().gd_weight_store_add(store.handle, b"x", buf.ctypes.data_as(C.c_void_p), N.GD_F16, shape, 1) \
        == N.GD_ERR_INVALID_ARGUMENT
