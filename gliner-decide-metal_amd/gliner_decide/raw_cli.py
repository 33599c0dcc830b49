"""`gliner-decide-raw` (RawCLI.swift:24-302): text (or a JSONL file of
examples) + decision tasks in, label predictions out, on the HIP classifier.

    python -m gliner_decide.raw_cli --text TEXT --tasks schema.json
    python -m gliner_decide.raw_cli --jsonl examples.jsonl --output results.json
        [--tokenizer DIR] [--weights FILE] [--buckets 32,64,...] [--batch-size N]

JSONL mode (RawCLI.swift:104-171): every line `{"id", "text", "tasks"}` is
formatted and tokenized (timed per line), the rows are grouped by their
(L, Hh, O) shape, each group runs in batches of `--batch-size` rows, every
row is decoded with its own tasks, and the results come out in input order
as one JSON array of `{id, predictions, preprocessingMilliseconds,
inferenceMilliseconds}` (a batch's forward time shared evenly by its rows).
Batches are launched while later lines are still being tokenized.

Single mode (:60-102): one text against the tasks of `--tasks`, the
predictions printed as JSON, preprocessing and inference milliseconds on
stderr; `--dump-input FILE` saves the four input arrays as safetensors.
"""

from __future__ import annotations

import argparse
import json
import re
import sys
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .decode import DEFAULT_BUCKETS, decode, row_extents
from .frontend import NativeDecisionTokenizer, tasks_from_json


@dataclass
class RawExample:  # RawCLI.swift:11-15
    id: str
    text: str
    tasks: list

    @classmethod
    def from_json(cls, obj) -> "RawExample":
        if not isinstance(obj, dict):
            raise ValueError("a JSONL example is an object {\"id\", \"text\", \"tasks\"}")
        missing = [k for k in ("id", "text", "tasks") if k not in obj]
        if missing:
            raise ValueError(f"example is missing {', '.join(missing)}")
        if not isinstance(obj["id"], str) or not isinstance(obj["text"], str):
            raise ValueError("example id and text must be strings")
        if not isinstance(obj["tasks"], list):
            raise ValueError("example tasks must be a list")
        return cls(obj["id"], obj["text"], tasks_from_json(obj["tasks"]))


@dataclass
class _Pending:  # RawCLI.swift:225-230
    index: int
    example: RawExample
    input: object
    preprocessing_ms: float


def _host_logits(logits) -> np.ndarray:
    """[B, Hh, O] logits as fp32 on the host (RawCLI.swift:152-153)."""
    if hasattr(logits, "cpu"):
        return logits.float().cpu().numpy()
    return np.asarray(logits, np.float32)


def _concat(inputs):
    """Stacks one-row inputs; marker arrays are padded to the batch's largest
    Hh and O with masked slots (index 0, mask 0), which the head fills with
    -10000 and decode never reads."""
    from .classifier import DecisionInput
    hh = max(x.marker_indices.shape[1] for x in inputs)
    oo = max(x.marker_indices.shape[2] for x in inputs)

    def pad(a):
        a = np.asarray(a)
        if a.shape[1:] == (hh, oo):
            return a
        out = np.zeros((a.shape[0], hh, oo), a.dtype)
        out[:, :a.shape[1], :a.shape[2]] = a
        return out

    return DecisionInput(np.concatenate([np.asarray(x.input_ids) for x in inputs], axis=0),
                         np.concatenate([np.asarray(x.attention_mask) for x in inputs], axis=0),
                         np.concatenate([pad(x.marker_indices) for x in inputs], axis=0),
                         np.concatenate([pad(x.marker_mask) for x in inputs], axis=0))


def parse_jsonl(text: str) -> list:
    """Non-empty lines of a JSONL document as RawExamples (a line that does
    not parse is an error naming its line)."""
    return list(iter_jsonl(text.splitlines()))


def iter_jsonl(lines):
    for n, line in enumerate(lines, 1):
        if not line.strip():
            continue
        try:
            yield RawExample.from_json(json.loads(line))
        except ValueError as e:
            raise ValueError(f"line {n}: {e}") from None


class _HostBatches:
    """Runs each batch with `model.classify` (synchronous), for models that
    take host arrays only."""

    def __init__(self, model):
        self.model = model
        self.done = []

    def submit(self, inp, rows) -> None:
        result = self.model.classify(inp)
        self.done.append((rows, _host_logits(result.logits), result.wall_milliseconds))

    def ready(self) -> list:
        done, self.done = self.done, []
        return done

    def finish(self) -> list:
        return self.ready()


class _DeviceBatches:
    """Enqueues each batch on the current stream without waiting for the GPU:
    inputs go up from pinned host memory, the forward is bracketed by two HIP
    events, and the logits come back into pinned host memory behind a third,
    so the host keeps tokenizing and decodes each batch once its last event
    has completed.  The workspace grows (a device synchronisation) only when a
    batch needs more than was reserved."""

    def __init__(self, model, tokens: int, markers: int):
        import torch
        self.torch = torch
        self.model = model
        self.device = torch.device("cuda", torch.cuda.current_device())
        self.jobs = []
        self.tokens, self.markers = tokens, markers
        model.reserve(1, tokens, 1, markers)

    def submit(self, inp, rows) -> None:
        torch = self.torch
        B, L, Hh, O = inp.shape
        if B * L > self.tokens or B * Hh * O > self.markers:
            self.tokens, self.markers = max(self.tokens, B * L), max(self.markers, 2 * B * Hh * O)
            self.model.reserve(1, self.tokens, 1, self.markers)
        up = [torch.from_numpy(np.ascontiguousarray(getattr(inp, f))).pin_memory().to(self.device, non_blocking=True)
              for f in ("input_ids", "attention_mask", "marker_indices", "marker_mask")]
        out = torch.empty((B, Hh, O), dtype=torch.float16, device=self.device)
        host = torch.empty((B, Hh, O), dtype=torch.float16, pin_memory=True)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)] + [torch.cuda.Event()]
        total = None
        if not getattr(self.model, "full_rows", False):
            total = int(row_extents(inp.attention_mask, inp.marker_indices, inp.marker_mask).sum())
        ev[0].record()
        self.model.classify_device(*up, out, total_tokens=total)
        ev[1].record()
        host.copy_(out, non_blocking=True)
        ev[2].record()
        self.jobs.append((rows, up, out, host, ev))

    def _take(self, n) -> list:
        done = [(rows, host.float().numpy(), ev[0].elapsed_time(ev[1])) for rows, _, _, host, ev in self.jobs[:n]]
        del self.jobs[:n]
        return done

    def ready(self) -> list:
        n = 0
        while n < len(self.jobs) and self.jobs[n][4][2].query():
            n += 1
        return self._take(n)

    def finish(self) -> list:
        self.torch.cuda.current_stream().synchronize()
        return self._take(len(self.jobs))


def run_examples(examples, frontend, model, buckets=DEFAULT_BUCKETS, batch_size: int = 32, log=None,
                 total: int | None = None, group_by_length: bool = True) -> list:
    """RawCLI.swift:112-164 on examples (any iterable): returns the result
    objects in input order.

    Rows are grouped in input order and each group is cut into runs of
    `batch_size`; a batch is launched as soon as its group has filled it (the
    rest of each group at the end), so tokenization overlaps the forward
    passes.  group_by_length=False groups by (L, Hh, O) exactly as the
    reference does; the default groups by L only, padding each batch's marker
    arrays to its largest Hh and O with masked slots: a row's logits depend on
    its own ids and markers only, so the decisions are the same and fewer
    batches run part-full.

    With a model that has `classify_device` (the HIP classifier) batches are
    enqueued asynchronously, decoded as they complete, and
    `inferenceMilliseconds` is the batch's GPU forward time (HIP events)
    divided by its rows; otherwise `model.classify(DecisionInput) ->
    InferenceResult` runs each batch and its wall time is shared."""
    if batch_size < 1:
        raise ValueError("batch size must be at least 1")
    if hasattr(model, "classify_device"):
        runner = _DeviceBatches(model, batch_size * max(max(buckets, default=32), 32), batch_size * 64)
    else:
        runner = _HostBatches(model)
    groups: dict = {}
    results: dict = {}

    def collect(done):
        for rows, logits, ms in done:
            per_row = ms / len(rows)
            for row, it in enumerate(rows):
                results[it.index] = {
                    "id": it.example.id,
                    "predictions": [p.to_json() for p in decode(logits, row, it.example.tasks)],
                    "preprocessingMilliseconds": it.preprocessing_ms,
                    "inferenceMilliseconds": per_row,
                }

    count = 0
    for index, ex in enumerate(examples):
        t0 = time.perf_counter_ns()
        inp = frontend.make_input(ex.text, ex.tasks, buckets)
        item = _Pending(index, ex, inp, (time.perf_counter_ns() - t0) / 1e6)
        count = index + 1
        if log is not None and total is not None and (count % 100 == 0 or count == total):
            log(f"tokenized {count}/{total}")
        _, L, Hh, O = inp.shape
        group = groups.setdefault(L if group_by_length else (L, Hh, O), [])
        group.append(item)
        if len(group) == batch_size:
            runner.submit(_concat([it.input for it in group]), group[:])
            group.clear()
            collect(runner.ready())
    if log is not None and total is None:
        log(f"tokenized {count}/{count}")
    for group in groups.values():
        if group:
            runner.submit(_concat([it.input for it in group]), group)
    collect(runner.finish())
    return [results[i] for i in range(count)]


def run_jsonl(path, frontend, model, buckets=DEFAULT_BUCKETS, batch_size: int = 32, output=None, log=None) -> list:
    """RawCLI.swift:104-171: reads the JSONL file, runs it, writes the JSON
    array to `output` (or prints it)."""
    lines = Path(path).read_text(encoding="utf-8").splitlines()
    total = sum(1 for line in lines if line.strip())
    results = run_examples(iter_jsonl(lines), frontend, model, buckets, batch_size, log, total)
    data = json.dumps(results, separators=(",", ":"))
    if output is not None:
        Path(output).write_text(data, encoding="utf-8")
    else:
        print(data)
    return results


def run_single(text: str, tasks, frontend, model, buckets=DEFAULT_BUCKETS, dump_input=None, err=sys.stderr) -> list:
    """RawCLI.swift:60-102; returns the predictions and prints them."""
    t0 = time.perf_counter_ns()
    inp = frontend.make_input(text, tasks, buckets)
    pre_ms = (time.perf_counter_ns() - t0) / 1e6
    if dump_input is not None:
        from safetensors.numpy import save_file
        save_file({"input_ids": np.asarray(inp.input_ids), "attention_mask": np.asarray(inp.attention_mask),
                   "marker_indices": np.asarray(inp.marker_indices), "marker_mask": np.asarray(inp.marker_mask)},
                  str(dump_input))
    result = model.classify(inp)
    preds = [p.to_json() for p in decode(_host_logits(result.logits), 0, tasks)]
    print(json.dumps(preds, separators=(",", ":")))
    err.write(f"preprocessing_ms: {pre_ms:.3f}\n")
    err.write(f"inference_ms: {result.wall_milliseconds:.3f}\n")
    return preds


def parse_args(argv=None):
    """Options (RawCLI.swift:232-301), the same names and defaults."""
    p = argparse.ArgumentParser(prog="gliner-decide-raw",
                                description="GLiNER-Decide classification on the MI355X HIP encoder")
    p.add_argument("--text")
    p.add_argument("--tasks", default="Artifacts/tasks.json")
    p.add_argument("--jsonl")
    p.add_argument("--tokenizer", default="Artifacts/coreml-runtime")
    p.add_argument("--weights", default="Artifacts/decide-classification-fp16.safetensors")
    p.add_argument("--buckets", default=",".join(str(b) for b in DEFAULT_BUCKETS))
    p.add_argument("--batch-size", default="32")
    p.add_argument("--dump-input")
    p.add_argument("--output")
    p.add_argument("--generic-attention", action="store_true")
    p.add_argument("--fused-attention-kernel", action="store_true")
    a = p.parse_args(argv)
    if a.text is None and a.jsonl is None:
        p.error("--text or --jsonl is required")
    # Swift `split(",").compactMap { Int($0) }`: pieces that are not integers drop out
    a.batch_size = int(a.batch_size) if re.fullmatch(r"[+-]?[0-9]+", a.batch_size) else 32
    a.buckets = [int(x) for x in a.buckets.split(",") if re.fullmatch(r"[+-]?[0-9]+", x)]
    return a


def main(argv=None) -> int:
    a = parse_args(argv)
    try:
        from .classifier import GLiNERDecideClassifier
        frontend = NativeDecisionTokenizer(a.tokenizer)
        model = GLiNERDecideClassifier(a.weights, use_compiled_graph=True, use_fast_attention=not a.generic_attention,
                                       use_custom_relative_kernel=False,
                                       use_fused_attention_kernel=a.fused_attention_kernel)
        if a.jsonl is not None:
            run_jsonl(a.jsonl, frontend, model, a.buckets, a.batch_size, a.output,
                      log=lambda m: sys.stderr.write(m + "\n"))
        else:
            tasks = tasks_from_json(json.loads(Path(a.tasks).read_text(encoding="utf-8")))
            run_single(a.text, tasks, frontend, model, a.buckets, a.dump_input)
    except Exception as e:  # RawCLI.swift:54-57
        sys.stderr.write(f"error: {e}\n")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
