"""`gliner-decide-metal` (main.swift): the batch / latency driver over the HIP
classifier, with the reference's options, defaults and printed lines.

    python -m gliner_decide.metal_cli --weights W.safetensors --inputs I.safetensors
        [--warmup 3] [--iterations 20] [--profile] [--fused] [--compiled]
        [--batch-size N [--pad-batch]] [--output logits.safetensors]
    python -m gliner_decide.metal_cli --kernel-test | --relative-kernel-test

* `--kernel-test` / `--relative-kernel-test` (main.swift:141-225) run the fused
  residual LayerNorm / relative-bias kernels on the reference's procedural
  inputs and print expected (the reference's formula evaluated on the host
  with its fp16 rounding points), actual (the GPU kernel) and max_abs; they
  need no weights.
* `--batch-size N` (main.swift:243-285): all rows of the input file in chunks
  of N (the last one padded with copies of its last row under --pad-batch,
  main.swift:7-51), warm-up chunks first, then batch_count, batch_total_ms and
  batch_rows_per_sec; `--output` saves the concatenated logits.
* otherwise (main.swift:287-320): --warmup + --iterations classify calls of the
  whole input, p50 / p95 / mean wall milliseconds, the per-stage profile under
  --profile, the last logits under --output.

The model shape (layers, vocabulary) is read from the weights file; the real
checkpoint gives DeBERTaV2Configuration.default (Configuration.swift:38-48).
"""

from __future__ import annotations

import dataclasses
import json
import re
import struct
import sys
import time
from pathlib import Path

import numpy as np

_INT = re.compile(r"[+-]?[0-9]+")

FLAGS = {"--profile": "profile", "--fused": "fused", "--kernel-test": "kernel_test",
         "--relative-kernel-test": "relative_kernel_test", "--compiled": "compiled",
         "--custom-relative": "custom_relative", "--fused-attention-kernel": "fused_attention_kernel",
         "--pad-batch": "pad_batch"}
VALUES = {"--weights": "weights", "--inputs": "inputs", "--output": "output"}
INTS = {"--warmup": "warmup", "--iterations": "iterations", "--batch-size": "batch_size"}

USAGE = """GLiNER2.5-Decide classification-only HIP benchmark (MI355X)

--weights PATH     FP16 classification weights
--inputs PATH      safetensors containing input_ids, attention_mask,
                    marker_indices, marker_mask
--warmup N         warmup iterations (default: 3)
--iterations N     measured iterations (default: 20)
--profile          evaluate and print per-stage timings
--fused            residual LayerNorm with the sum kept in fp32
--kernel-test      compare the fused residual LayerNorm kernel with the LayerNorm formula
--relative-kernel-test
                   compare the relative-bias kernel with the reference's ops
--compiled         capture and replay the forward as a HIP graph
--fast-attention   fused attention (default)
--generic-attention
                   the explicit score path (not built: exits with an error)
--custom-relative / --fused-attention-kernel
                   accepted; the fused attention kernel is the only path
--batch-size N     process all rows in input file in chunks of N
--pad-batch        pad the final partial chunk to the full batch size
--output PATH      write logits as safetensors"""


class Options:
    """main.swift:52-103: the same names and defaults; an integer option that
    does not parse keeps its default (Swift `Int(x) ?? default`)."""

    def __init__(self, argv):
        self.weights = "Artifacts/decide-classification-fp16.safetensors"
        self.inputs = "Artifacts/sample-inputs.safetensors"
        self.warmup, self.iterations, self.batch_size = 3, 20, 0
        self.output = None
        self.fast_attention = True
        self.help = False
        for f in FLAGS.values():
            setattr(self, f, False)
        i = 0
        while i < len(argv):
            a = argv[i]

            def value():
                if i + 1 >= len(argv):
                    raise SystemExit(f"Missing value for {a}")
                return argv[i + 1]

            if a in VALUES:
                setattr(self, VALUES[a], value())
                i += 1
            elif a in INTS:
                v = value()
                if _INT.fullmatch(v):
                    setattr(self, INTS[a], int(v))
                i += 1
            elif a in FLAGS:
                setattr(self, FLAGS[a], True)
            elif a == "--fast-attention":
                self.fast_attention = True
            elif a == "--generic-attention":
                self.fast_attention = False
            elif a in ("--help", "-h"):
                self.help = True
                break
            else:
                raise SystemExit(f"Unknown argument: {a}")
            i += 1


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def relative_test_case() -> dict:
    """main.swift:143-174: b=1, h=2, l=8, d=4, p=8 procedural inputs and index
    tensors, and the expected value of the reference's op chain, every op
    rounded to fp16 as MLX does: where(mask > -60000, (takeAlong(q posK^T,
    c2p) + takeAlong(k posQ^T, p2c)^T) / fp16(sqrt(3d)), -65504)."""
    b, h, l, d, p = 1, 2, 8, 4, 8
    q = _f16([(i % 13) / 13.0 for i in range(b * h * l * d)]).reshape(b, h, l, d)
    k = _f16([((i * 7) % 17) / 17.0 for i in range(b * h * l * d)]).reshape(b, h, l, d)
    pk = _f16([((i * 3) % 19) / 19.0 for i in range(h * p * d)]).reshape(1, h, p, d)
    pq = _f16([((i * 5) % 23) / 23.0 for i in range(h * p * d)]).reshape(1, h, p, d)
    c2p = np.array([i % p for i in range(h * l * l)], np.int32).reshape(1, h, l, l)
    p2c = np.array([(i * 3) % p for i in range(h * l * l)], np.int32).reshape(1, h, l, l)
    mask = _f16([0.0 if i < 6 else -65504.0 for i in range(l)]).reshape(1, 1, 1, l)
    scale = float(np.float32(np.sqrt(d * 3)))
    raw_c2p = (q.astype(np.float32) @ np.swapaxes(pk, -1, -2).astype(np.float32)).astype(np.float16)
    raw_p2c = (k.astype(np.float32) @ np.swapaxes(pq, -1, -2).astype(np.float32)).astype(np.float16)
    e_c2p = np.take_along_axis(raw_c2p, np.broadcast_to(c2p, (b, h, l, l)), -1)
    e_p2c = np.swapaxes(np.take_along_axis(raw_p2c, np.broadcast_to(p2c, (b, h, l, l)), -1), -1, -2)
    summed = (e_c2p.astype(np.float32) + e_p2c.astype(np.float32)).astype(np.float16)
    rel = (summed.astype(np.float32) / np.float32(np.float16(scale))).astype(np.float16)
    expected = np.where(mask > np.float16(-60000.0), rel, np.float16(-65504.0)).astype(np.float16)
    return dict(q=q, k=k, position_key=pk, position_query=pq, c2p=c2p, p2c=p2c, mask=mask, scale=scale,
                dims=(b, h, l, d, p), expected=expected)


def layer_norm_test_case() -> dict:
    """main.swift:195-211: x = i / 1024 for i < 1024, residual 0, weight 1,
    bias 0, eps 1e-7, and the expected MLXFast.layerNorm(x + residual):
    biased variance in fp32, one rounding to fp16 at the output."""
    x = _f16(np.arange(1024) / 1024.0).reshape(1, 1, 1024)
    residual = np.zeros((1, 1, 1024), np.float16)
    weight = np.ones(1024, np.float16)
    bias = np.zeros(1024, np.float16)
    summed = (x.astype(np.float32) + residual.astype(np.float32)).astype(np.float16)
    s32 = summed.astype(np.float32)
    mean = s32.mean(-1, keepdims=True)
    var = ((s32 - mean) ** 2).mean(-1, keepdims=True)
    expected = ((s32 - mean) / np.sqrt(var + np.float32(1e-7)) * weight + bias).astype(np.float16)
    return dict(x=x, residual=residual, weight=weight, bias=bias, summed=summed, eps=1e-7, expected=expected)


def _report(expected, actual, out) -> float:
    max_abs = float(np.max(np.abs(expected.astype(np.float32) - actual.astype(np.float32))))
    out(f"expected: {expected}")
    out(f"actual:   {actual}")
    out(f"max_abs:  {max_abs}")
    return max_abs


def relative_kernel_test(out=print) -> float:
    """--relative-kernel-test (main.swift:141-192): the general-index
    relative-bias kernel on relative_test_case(), printed beside the
    expected value."""
    import torch
    from .device import require_gpu
    from .fused_kernels import FusedKernels
    case = relative_test_case()
    dev = require_gpu()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    b, h, l, d, p = case["dims"]
    actual = FusedKernels().relative_bias(t(case["q"]), t(case["k"]), t(case["position_key"]),
                                          t(case["position_query"]), t(case["c2p"]), t(case["p2c"]),
                                          t(case["mask"]), 1.0 / case["scale"], b, h, l, d, p)
    return _report(case["expected"], actual.cpu().numpy(), out)


def kernel_test(out=print) -> float:
    """--kernel-test (main.swift:194-225): the fused residual LayerNorm (sum
    kept in fp32, as the reference's kernel) on layer_norm_test_case()."""
    import torch
    from .device import require_gpu
    from .fused_kernels import FusedKernels
    case = layer_norm_test_case()
    out(f"input:    {case['x']}")
    out(f"residual: {case['residual']}")
    out(f"summed:   {case['summed']}")
    dev = require_gpu()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    actual = FusedKernels().residual_layer_norm(t(case["x"]), t(case["residual"]), t(case["weight"]),
                                                t(case["bias"]), case["eps"])
    return _report(case["expected"], actual.cpu().numpy(), out)


def config_from_weights(path):
    """DeBERTaV2Configuration.default with the layer count and vocabulary of
    the checkpoint's tensors (read from the safetensors header only)."""
    from .config import DeBERTaV2Configuration
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
    cfg = DeBERTaV2Configuration.default()
    emb = header.get("encoder.embeddings.word_embeddings.weight")
    if emb:
        cfg = dataclasses.replace(cfg, vocab_size=int(emb["shape"][0]))
    layers = {int(m.group(1)) for k in header for m in [re.match(r"encoder\.encoder\.layer\.(\d+)\.", k)] if m}
    if layers:
        cfg = dataclasses.replace(cfg, num_hidden_layers=max(layers) + 1)
    return cfg


def run(o: Options, out=print) -> dict:
    import torch
    from safetensors.numpy import save_file
    from .classifier import DecisionInput, GLiNERDecideClassifier
    from .decode import make_batch_chunk
    if o.relative_kernel_test:
        return {"max_abs": relative_kernel_test(out)}
    if o.kernel_test:
        return {"max_abs": kernel_test(out)}
    model = GLiNERDecideClassifier(o.weights, config_from_weights(o.weights), use_fused_kernels=o.fused,
                                   use_compiled_graph=o.compiled, use_fast_attention=o.fast_attention,
                                   use_custom_relative_kernel=o.custom_relative,
                                   use_fused_attention_kernel=o.fused_attention_kernel)
    inp = DecisionInput.from_safetensors(o.inputs)
    out(f"device: {torch.cuda.get_device_name(0)}")
    out(f"weights: {Path(o.weights).resolve()}")
    out(f"inputs: {Path(o.inputs).resolve()}")
    arrays = {k: np.asarray(getattr(inp, k)) for k in ("input_ids", "attention_mask", "marker_indices",
                                                        "marker_mask")}
    if o.batch_size > 0:
        count = arrays["input_ids"].shape[0]
        if count == 0:
            raise SystemExit("batch input must contain at least one row")
        if max(0, o.warmup) > 0:
            warm_end = min(o.batch_size, count)
            warm, _ = make_batch_chunk(arrays, 0, warm_end, o.batch_size if o.pad_batch else warm_end)
            for _ in range(max(1, o.warmup)):
                model.classify(DecisionInput(**warm))
        started = time.perf_counter_ns()
        pieces = []
        offset = 0
        while offset < count:
            end = min(offset + o.batch_size, count)
            chunk, valid = make_batch_chunk(arrays, offset, end, o.batch_size if o.pad_batch else end - offset)
            pieces.append(model.classify(DecisionInput(**chunk)).logits[:valid])
            offset = end
        logits = torch.cat(pieces, 0).cpu().numpy()
        elapsed = time.perf_counter_ns() - started
        out(f"batch_count: {count}")
        out(f"batch_total_ms: {elapsed / 1e6:.3f}")
        out(f"batch_rows_per_sec: {count / (elapsed / 1e9):.3f}")
        if o.output:
            save_file({"logits": logits}, o.output)
            out(f"output: {o.output}")
        return {"logits": logits, "rows_per_sec": count / (elapsed / 1e9)}
    for _ in range(max(0, o.warmup)):
        model.classify(inp)
    timings, last = [], None
    for _ in range(max(1, o.iterations)):
        last = model.classify(inp, collect_profile=o.profile)
        timings.append(last.wall_milliseconds)
    srt = sorted(timings)
    p50 = srt[len(srt) // 2]
    p95 = srt[min(len(srt) - 1, int((len(srt) - 1) * 0.95))]
    out(f"p50_ms: {p50:.3f}")
    out(f"p95_ms: {p95:.3f}")
    out(f"mean_ms: {sum(timings) / len(timings):.3f}")
    if o.profile:
        out("profile:")
        for ev in last.events:
            out(f"  {ev.name:<42s} {ev.milliseconds:8.3f} ms")
    logits = last.logits.cpu().numpy()
    if o.output:
        save_file({"logits": logits}, o.output)
        out(f"output: {o.output}")
    return {"logits": logits, "p50_ms": p50}


def main(argv=None) -> int:
    o = Options(sys.argv[1:] if argv is None else argv)
    if o.help:
        print(USAGE)
        return 0
    try:
        run(o)
    except SystemExit:
        raise
    except Exception as e:
        sys.stderr.write(f"error: {e}\n")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
