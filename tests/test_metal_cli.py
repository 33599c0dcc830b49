"""The `gliner-decide-metal` driver mirror (main.swift): option parsing, the
two known-answer self-tests, the batch and latency modes."""

import numpy as np
import pytest

from oracle import deberta as O


def _options(argv):
    from gliner_decide.metal_cli import Options
    return Options(argv)


def test_options_defaults_and_swift_int_parsing():
    """main.swift:52-103: defaults; `Int(x) ?? default` keeps the default on a
    value that is not an integer; --generic-attention clears fast attention;
    --help stops the parse where it stands."""
    o = _options([])
    assert (o.weights, o.inputs) == ("Artifacts/decide-classification-fp16.safetensors",
                                     "Artifacts/sample-inputs.safetensors")
    assert (o.warmup, o.iterations, o.batch_size, o.output) == (3, 20, 0, None)
    assert o.fast_attention and not (o.profile or o.fused or o.compiled or o.pad_batch)
    o = _options(["--warmup", "x", "--iterations", "+7", "--batch-size", "-2", "--pad-batch", "--profile",
                  "--fused", "--compiled", "--generic-attention", "--output", "o.safetensors"])
    assert (o.warmup, o.iterations, o.batch_size) == (3, 7, -2)
    assert o.pad_batch and o.profile and o.fused and o.compiled and not o.fast_attention
    assert o.output == "o.safetensors"
    o = _options(["--generic-attention", "--fast-attention", "--custom-relative", "--fused-attention-kernel"])
    assert o.fast_attention and o.custom_relative and o.fused_attention_kernel
    o = _options(["-h", "--not-an-option"])
    assert o.help


@pytest.mark.parametrize("argv,message", [(["--bogus"], "Unknown argument: --bogus"),
                                          (["--weights"], "Missing value for --weights"),
                                          (["--warmup"], "Missing value for --warmup")])
def test_options_errors(argv, message):
    with pytest.raises(SystemExit, match=message):
        _options(argv)


def test_help_prints_usage(capsys):
    from gliner_decide.metal_cli import main
    assert main(["--help"]) == 0
    text = capsys.readouterr().out
    for flag in ("--weights", "--inputs", "--kernel-test", "--relative-kernel-test", "--batch-size", "--pad-batch",
                 "--output"):
        assert flag in text


def test_relative_test_case_against_oracle_kernel():
    """The reference's op-chain expectation (three fp16 roundings) sits within
    two fp16 ulp of the oracle's single-rounding kernel restatement on the
    same procedural inputs; the masked keys (l >= 6) hold -65504 exactly.  A
    p2c gather without its transpose moves entries by far more than that."""
    from gliner_decide.metal_cli import relative_test_case
    c = relative_test_case()
    b, h, l, d, p = c["dims"]
    want = O.relative_bias_kernel(c["q"], c["k"], c["position_key"], c["position_query"], c["c2p"].reshape(h, l, l),
                                  c["p2c"].reshape(h, l, l), c["mask"].reshape(b, l), 1.0 / c["scale"])
    got = c["expected"].astype(np.float32)
    assert np.all(got[..., 6:] == -65504.0)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want[..., :6]), 2.0 ** -14))) - 10)
    assert np.all(np.abs(got[..., :6] - want[..., :6]) <= 2 * ulp)
    wrong = O.relative_bias_kernel(c["q"], c["k"], c["position_key"], c["position_query"], c["c2p"].reshape(h, l, l),
                                   np.swapaxes(c["p2c"].reshape(h, l, l), 1, 2), c["mask"].reshape(b, l),
                                   1.0 / c["scale"])
    assert np.max(np.abs(wrong[..., :6] - got[..., :6])) > 0.05


def test_layer_norm_test_case_against_oracle_and_closed_form():
    """x_i = i / 1024: mean 1023/2048 and variance (1024^2 - 1) / (12 * 1024^2)
    in closed form; the expectation equals the oracle's fused-kernel LN."""
    from gliner_decide.metal_cli import layer_norm_test_case
    c = layer_norm_test_case()
    want = O.residual_layer_norm_kernel(c["x"], c["residual"], c["weight"], c["bias"], c["eps"])
    assert np.array_equal(c["expected"], want.astype(np.float16))
    i = np.arange(1024, dtype=np.float64)
    closed = (i / 1024 - 1023 / 2048) / np.sqrt((1024 ** 2 - 1) / (12 * 1024 ** 2) + 1e-7)
    assert np.max(np.abs(c["expected"].reshape(-1).astype(np.float64) - closed)) <= 2.0 ** -10


def test_config_from_weights_header(tmp_path):
    from safetensors.numpy import save_file
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.metal_cli import config_from_weights
    cfg = DeBERTaV2Configuration(num_hidden_layers=3, vocab_size=77, hidden_size=64, intermediate_size=128,
                                 num_attention_heads=4, classifier_hidden=32)
    from gliner_decide.synthetic import weight_shapes
    save_file({k: np.zeros(s, np.float16) for k, s in weight_shapes(cfg).items()}, tmp_path / "w.safetensors")
    got = config_from_weights(tmp_path / "w.safetensors")
    assert (got.num_hidden_layers, got.vocab_size) == (3, 77)
    assert got.hidden_size == DeBERTaV2Configuration.default().hidden_size


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
@pytest.mark.gpu
def test_kernel_self_tests_print_known_answers():
    """--kernel-test / --relative-kernel-test through the HIP kernels: the
    LayerNorm within one fp16 ulp of its largest output (|y| < 1.74), the
    relative bias within two ulp of its three-rounding expectation (|y| < 1)."""
    from gliner_decide.metal_cli import Options, run
    lines = []
    ln = run(Options(["--kernel-test"]), out=lines.append)["max_abs"]
    assert ln <= 2.0 ** -10
    assert [s.split(":")[0] for s in lines] == ["input", "residual", "summed", "expected", "actual", "max_abs"]
    lines.clear()
    rel = run(Options(["--relative-kernel-test"]), out=lines.append)["max_abs"]
    assert rel <= 2.0 ** -10
    assert [s.split(":")[0] for s in lines] == ["expected", "actual", "max_abs"]


def _small_files(tmp_path):
    from safetensors.numpy import save_file
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import classification_batch, synthetic_weights
    cfg = DeBERTaV2Configuration(num_hidden_layers=2, vocab_size=3000)
    save_file(synthetic_weights(cfg, seed=9), tmp_path / "w.safetensors")
    bt = classification_batch(seed=3, batch=5, seq_len=64, vocab=3000, min_len=12)
    ids = np.where(bt.input_ids >= 3000, bt.input_ids % 3000, bt.input_ids)  # marker ids past the vocabulary
    save_file({"input_ids": ids.astype(np.int64), "attention_mask": bt.attention_mask.astype(np.int64),
               "marker_indices": bt.marker_indices.astype(np.int64), "marker_mask": bt.marker_mask.astype(np.float32)},
              tmp_path / "in.safetensors")
    return cfg, bt


@pytest.mark.gpu
@pytest.mark.parametrize("pad", [False, True])
def test_batch_mode_matches_one_classify(tmp_path, pad):
    """--batch-size 2 over 5 rows (chunks 2, 2, 1; the last padded to 2 with
    copies of its last row under --pad-batch): the concatenated logits equal
    one classify of all rows within the probability-logit tolerance, and the
    --output file holds them."""
    from safetensors.numpy import load_file
    from gliner_decide import DecisionInput, GLiNERDecideClassifier
    from gliner_decide.metal_cli import Options, run
    cfg, bt = _small_files(tmp_path)
    argv = ["--weights", str(tmp_path / "w.safetensors"), "--inputs", str(tmp_path / "in.safetensors"),
            "--batch-size", "2", "--warmup", "1", "--output", str(tmp_path / "out.safetensors")]
    lines = []
    res = run(Options(argv + (["--pad-batch"] if pad else [])), out=lines.append)
    keys = [s.split(":")[0] for s in lines]
    assert keys[-4:] == ["batch_count", "batch_total_ms", "batch_rows_per_sec", "output"]
    assert lines[keys.index("batch_count")] == "batch_count: 5"
    got = load_file(str(tmp_path / "out.safetensors"))["logits"]
    assert got.shape == bt.marker_indices.shape and np.array_equal(got, res["logits"])
    model = GLiNERDecideClassifier(str(tmp_path / "w.safetensors"), cfg)
    want = model.classify(DecisionInput.from_safetensors(tmp_path / "in.safetensors")).logits.float().cpu().numpy()
    assert np.max(np.abs(got.astype(np.float32) - want)) <= 2e-3


@pytest.mark.gpu
def test_latency_mode_profile_and_output(tmp_path):
    """--iterations 3 --profile --compiled --fused: p50/p95/mean lines, the
    per-stage profile, and the last call's logits in --output."""
    from safetensors.numpy import load_file
    from gliner_decide.metal_cli import Options, run
    _small_files(tmp_path)
    argv = ["--weights", str(tmp_path / "w.safetensors"), "--inputs", str(tmp_path / "in.safetensors"),
            "--iterations", "3", "--warmup", "1", "--profile", "--compiled", "--fused",
            "--output", str(tmp_path / "out.safetensors")]
    lines = []
    res = run(Options(argv), out=lines.append)
    keys = [s.split(":")[0] for s in lines]
    for k in ("device", "weights", "inputs", "p50_ms", "p95_ms", "mean_ms", "profile", "output"):
        assert k in keys
    assert res["p50_ms"] > 0
    stages = lines[keys.index("profile") + 1:keys.index("output")]
    assert stages and all(s.startswith("  ") and s.endswith(" ms") for s in stages)
    assert np.array_equal(load_file(str(tmp_path / "out.safetensors"))["logits"], res["logits"])
