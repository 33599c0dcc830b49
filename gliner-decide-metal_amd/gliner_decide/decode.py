"""Host-side rules around the encoder: label decode, batch chunking, buckets.

References: `decode` (RawCLI.swift:182-223), `makeBatchChunk`
(main.swift:7-51), bucket selection (NativeTokenizer.swift:85-88, 134-138)
and grouping by shape (RawCLI.swift:135-163).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

DEFAULT_BUCKETS = (32, 64, 96, 128, 256, 512)


@dataclass(frozen=True)
class DecisionTask:
    """A task head (NativeTokenizer.swift:25-44): its label names, whether it
    is multi-label, an optional prompt and optional per-label descriptions."""

    name: str
    labels: tuple
    multi_label: bool = False
    prompt: str | None = None
    label_descriptions: dict | None = None

    @classmethod
    def from_json(cls, obj: dict) -> "DecisionTask":
        """The reference's Codable form: `name`, `labels`, `multiLabel` are
        required, `prompt` and `labelDescriptions` optional."""
        missing = [k for k in ("name", "labels", "multiLabel") if k not in obj]
        if missing:
            raise ValueError(f"decision task is missing {', '.join(missing)}")
        if not isinstance(obj["name"], str):
            raise ValueError("decision task name must be a string")
        labels = obj["labels"]
        if not isinstance(labels, list) or not all(isinstance(x, str) for x in labels):
            raise ValueError("decision task labels must be a list of strings")
        if not isinstance(obj["multiLabel"], bool):
            raise ValueError("decision task multiLabel must be a boolean")
        desc = obj.get("labelDescriptions")
        if desc is not None and not (isinstance(desc, dict) and all(isinstance(v, str) for v in desc.values())):
            raise ValueError("decision task labelDescriptions must map labels to strings")
        prompt = obj.get("prompt")
        if prompt is not None and not isinstance(prompt, str):
            raise ValueError("decision task prompt must be a string")
        return cls(obj["name"], tuple(labels), obj["multiLabel"], prompt, desc)

    def to_json(self) -> dict:
        out = {"name": self.name, "labels": list(self.labels), "multiLabel": self.multi_label}
        if self.prompt is not None:
            out["prompt"] = self.prompt
        if self.label_descriptions is not None:
            out["labelDescriptions"] = dict(self.label_descriptions)
        return out


@dataclass
class Prediction:  # RawCLI.swift:5-9
    task: str
    labels: list
    probabilities: list

    def to_json(self) -> dict:
        return {"task": self.task, "labels": list(self.labels), "probabilities": list(self.probabilities)}


def decode(logits, row: int, tasks) -> list:
    """RawCLI.swift:182-223.  logits: [B, Hh, O] (any float type).
    Single-label: max-shifted softmax over the task's labels, argmax (first
    maximum).  Multi-label: sigmoid, labels with p >= 0.5, argmax if none."""
    arr = np.asarray(logits, dtype=np.float32)
    out = []
    for head, task in enumerate(tasks):
        probs = [float(arr[row, head, i]) for i in range(len(task.labels))]
        if task.multi_label:
            probs = [_sigmoid(x) for x in probs]
            selected = [i for i, p in enumerate(probs) if p >= 0.5]
            if not selected:
                selected = [_first_argmax(probs)]
            out.append(Prediction(task.name, [task.labels[i] for i in selected], probs))
        else:
            m = max(probs) if probs else 0.0
            ex = [math.exp(x - m) for x in probs]
            total = sum(ex)
            probs = [e / total for e in ex]
            best = _first_argmax(probs)
            out.append(Prediction(task.name, [task.labels[best]], probs))
    return out


def _sigmoid(x: float) -> float:
    """1 / (1 + exp(-x)) with IEEE overflow: Swift's Double exp returns +inf
    below x = -709.78 (probability 0), where math.exp raises."""
    e = math.exp(-x) if -x < 709.78 else math.inf
    return 1.0 / (1.0 + e)


def _first_argmax(values) -> int:
    """Swift `max(by:)` keeps the first of equal maxima."""
    best = 0
    for i, v in enumerate(values):
        if v > values[best]:
            best = i
    return best


def select_bucket(length: int, buckets=DEFAULT_BUCKETS) -> int:
    """Smallest bucket >= length (NativeTokenizer.swift:134-138)."""
    ordered = sorted(set(buckets))
    if not ordered:
        raise ValueError("no buckets")
    for b in ordered:
        if b >= length:
            return b
    raise ValueError(f"input of length {length} does not fit buckets {ordered}")


def make_batch_chunk(arrays: dict, start: int, end: int, pad_to: int):
    """main.swift:7-51: rows [start, end), padded to pad_to rows with copies
    of the last valid row.  Returns (chunk, valid_count)."""
    valid = end - start
    if valid <= 0:
        raise ValueError("empty chunk")
    chunk = {k: np.asarray(v)[start:end] for k, v in arrays.items()}
    if valid >= pad_to:
        return chunk, valid
    pad = pad_to - valid
    return {k: np.concatenate([v, np.repeat(v[valid - 1:valid], pad, axis=0)], axis=0) for k, v in chunk.items()}, valid


def row_extents(attention_mask, marker_indices, marker_mask) -> np.ndarray:
    """Per-row extents [B] (int64): the larger of (last l with
    attention_mask[b, l] > 0) + 1 and (last position read by a marker slot of
    row b with marker_mask > 0) + 1, where a marker outside [0, L) reads
    position 0; 0 for a row with neither.  Every position the classifier reads
    lies before the extent; its sum is the token count of packed rows."""
    mask = np.asarray(attention_mask, dtype=np.float32)
    B, L = mask.shape
    valid = mask > 0
    last = np.where(valid.any(axis=1), L - np.argmax(valid[:, ::-1], axis=1), 0)
    mi = np.asarray(marker_indices).reshape(B, -1).astype(np.int64)
    mm = np.asarray(marker_mask, dtype=np.float32).reshape(B, -1) > 0
    pos = np.where((mi >= 0) & (mi < L), mi + 1, 1)
    mark = np.where(mm, pos, 0).max(axis=1, initial=0)
    return np.maximum(last, mark).astype(np.int64)


def group_by_shape(items, key=lambda x: x):
    """RawCLI.swift:135-139: group requests by (L, Hh, O); insertion order."""
    groups: dict = {}
    for it in items:
        groups.setdefault(key(it), []).append(it)
    return groups
