"""Schema formatter and tokenizer front end: `NativeDecisionTokenizer`
(NativeTokenizer.swift:56-212) over the HF `tokenizers` Unigram model.

The reference runs the checkpoint's tokenizer.json through swift-transformers'
Unigram implementation (normaliser, Metaspace pre-tokenizer, Viterbi over the
piece scores); `tokenizers.Tokenizer.encode(..., add_special_tokens=False)` is
the same pipeline.  Everything around it is restated here:

* schema layout (NativeTokenizer.swift:91-116): per task
  `( [P] <prompt><descriptions> ( [L] label ... ) )`, tasks joined by
  `[SEP_STRUCT]`, then `[SEP_TEXT]` and the words of the text;
* word split (:193-208): a trailing `.` is added unless the text ends in
  `.`, `!` or `?` (`.` for an empty text), the word pattern below,
  case-insensitive, and every word lower-cased;
* entry tokenization (:159-191): every added token of tokenizer.json is cut
  out first (leftmost occurrence, the longer token on a tie) and maps to its
  id; the pieces between go through the tokenizer one entry at a time;
* marker positions (:123-130): the first token index of each `[L]` entry;
* bucket and padding (:131-157): the smallest requested bucket that holds the
  ids, right-padded with `[PAD]`; an fp16 0/1 attention mask; markers
  [1, Hh, O] with Hh = tasks, O = the largest label count, and an fp32 marker
  mask.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

import numpy as np
import regex

from .decode import DEFAULT_BUCKETS, DecisionTask

# NativeTokenizer.swift:69-72, an ICU (NSRegularExpression) pattern compiled
# case-insensitive.  ICU's classes are spelled out so that the `regex` module
# matches what ICU matches: \w = [\p{Alphabetic}\p{Mark}\p{Decimal_Number}
# \p{Connector_Punctuation}\u200c\u200d] (Python's \w has no combining marks)
# and \s = [\t\n\f\r\p{Z}].
_W = r"[\p{Alphabetic}\p{M}\p{Nd}\p{Pc}\u200c\u200d]"
_NS = r"[^\t\n\f\r\p{Z}]"
WORD_PATTERN = regex.compile(
    rf"(?:https?://{_NS}+|www\.{_NS}+)|[a-z0-9._%+-]+@[a-z0-9.-]+\.[a-z]{{2,}}|@[a-z0-9_]+|{_W}+(?:[-_]{_W}+)*|{_NS}",
    regex.IGNORECASE | regex.V0)


class TokenizerError(ValueError):
    """NativeTokenizerError (NativeTokenizer.swift:5-23)."""


def split_words(text: str) -> list:
    """NativeTokenizer.swift:193-208."""
    if not text:
        normalized = "."
    elif text[-1] in ".!?":
        normalized = text
    else:
        normalized = text + "."
    return [w.lower() for w in WORD_PATTERN.findall(normalized)]


def load_added_tokens(tokenizer_json: str | Path) -> dict:
    """`added_tokens` content -> id of a tokenizer.json (NativeTokenizer.swift:210-226)."""
    root = json.loads(Path(tokenizer_json).read_text(encoding="utf-8"))
    out = {}
    for tok in root.get("added_tokens") or []:
        content, tid = tok.get("content"), tok.get("id")
        if isinstance(content, str) and isinstance(tid, int):
            out[content] = tid
    return out


class NativeDecisionTokenizer:
    """Mirror of `NativeDecisionTokenizer` (NativeTokenizer.swift:56-75).

    `NativeDecisionTokenizer(directory)` reads tokenizer.json (and requires
    tokenizer_config.json beside it, as the reference does);
    `from_tokenizer(tokenizer, special_ids)` wraps a `tokenizers.Tokenizer`
    built in memory."""

    def __init__(self, directory: str | Path | None = None, *, tokenizer=None, special_ids: dict | None = None):
        if directory is not None:
            d = Path(directory)
            tj, cfg = d / "tokenizer.json", d / "tokenizer_config.json"
            if not (tj.is_file() and cfg.is_file()):
                raise TokenizerError(f"Tokenizer directory is missing tokenizer.json/tokenizer_config.json: {d}")
            try:
                json.loads(cfg.read_text(encoding="utf-8"))
            except ValueError as e:
                raise TokenizerError("Could not decode tokenizer_config.json") from e
            from tokenizers import Tokenizer
            tokenizer = Tokenizer.from_file(str(tj))
            special_ids = load_added_tokens(tj)
        if tokenizer is None:
            raise TokenizerError("a tokenizer directory or a tokenizers.Tokenizer is required")
        self.tokenizer = tokenizer
        self.special_ids = dict(special_ids or {})
        pad = self.special_ids.get("[PAD]")
        if pad is None:
            pad = tokenizer.token_to_id("[PAD]")
        self.pad_token_id = int(pad) if pad is not None else 0
        self.cache_size = 1 << 16
        self._cache: dict = {}
        # Leftmost occurrence, longest token first on a tie: an alternation
        # ordered by decreasing length picks exactly that (empty tokens never
        # match in the reference and are left out).
        toks = sorted((t for t in self.special_ids if t), key=lambda t: (-len(t), t))
        self._special_re = re.compile("|".join(re.escape(t) for t in toks)) if toks else None

    @classmethod
    def from_tokenizer(cls, tokenizer, special_ids: dict) -> "NativeDecisionTokenizer":
        return cls(tokenizer=tokenizer, special_ids=special_ids)

    # -- tokenization (NativeTokenizer.swift:159-191) --------------------------
    def _append_plain(self, text: str, ids: list) -> None:
        if text:
            ids.extend(self.tokenizer.encode(text, add_special_tokens=False).ids)

    def _entry_ids(self, text: str) -> tuple:
        ids: list = []
        if self._special_re is None:
            self._append_plain(text, ids)
            return tuple(ids)
        cursor = 0
        for m in self._special_re.finditer(text):
            if m.start() > cursor:
                self._append_plain(text[cursor:m.start()], ids)
            ids.append(self.special_ids[m.group(0)])
            cursor = m.end()
        self._append_plain(text[cursor:], ids)
        return tuple(ids)

    def append_tokenized(self, text: str, ids: list) -> None:
        # Every schema entry and word is tokenized on its own, and its ids are
        # a pure function of its text, so repeated entries (markers, labels,
        # prompts, frequent words) come from a bounded cache.
        hit = self._cache.get(text)
        if hit is None:
            hit = self._entry_ids(text)
            if len(self._cache) >= self.cache_size:
                self._cache.clear()
            self._cache[text] = hit
        ids.extend(hit)

    # -- schema (NativeTokenizer.swift:76-157) ---------------------------------
    @staticmethod
    def schema_entries(text: str, tasks) -> list:
        """(text, label-marker task index or None) entries of the schema and the
        text, in order."""
        groups = []
        for ti, task in enumerate(tasks):
            prompt = f"{task.name}: {task.prompt}" if task.prompt is not None else task.name
            descs = task.label_descriptions or {}
            descriptions = "".join(f" [DESCRIPTION] {label}: {descs[label]}" for label in task.labels
                                   if label in descs)
            entries = [("(", None), ("[P]", None), (prompt + descriptions, None), ("(", None)]
            for label in task.labels:
                entries.append(("[L]", ti))
                entries.append((label, None))
            entries += [(")", None), (")", None)]
            groups.append(entries)
        combined = []
        for ti, entries in enumerate(groups):
            combined += entries
            if ti < len(tasks) - 1:
                combined.append(("[SEP_STRUCT]", None))
        combined.append(("[SEP_TEXT]", None))
        combined += [(w, None) for w in split_words(text)]
        return combined

    def encode_ids(self, text: str, tasks) -> tuple:
        """Unpadded ids and the per-task marker positions."""
        ids: list = []
        markers = [[] for _ in tasks]
        for entry, marker in self.schema_entries(text, tasks):
            start = len(ids)
            self.append_tokenized(entry, ids)
            if marker is not None:
                markers[marker].append(start)
        return ids, markers

    def make_input(self, text: str, tasks, buckets=DEFAULT_BUCKETS):
        """`makeInput(text:tasks:buckets:)` -> DecisionInput of one row: input_ids
        [1, L] int32, attention_mask [1, L] fp16, marker_indices [1, Hh, O]
        int32, marker_mask [1, Hh, O] fp32."""
        from .classifier import DecisionInput
        tasks = list(tasks)
        if not tasks or not all(len(t.labels) > 0 for t in tasks):
            raise TokenizerError("Every decision task must contain at least one label")
        ordered = sorted(set(int(b) for b in buckets))
        if not ordered:
            raise TokenizerError(f"Encoded schema/text does not fit any requested bucket: {list(buckets)}")
        ids, markers = self.encode_ids(text, tasks)
        n = len(ids)
        bucket = next((b for b in ordered if b >= n), None)
        if bucket is None:
            raise TokenizerError(f"Encoded schema/text does not fit any requested bucket: {ordered}")
        input_ids = np.full((1, bucket), self.pad_token_id, dtype=np.int32)
        input_ids[0, :n] = ids
        mask = np.zeros((1, bucket), dtype=np.float16)
        mask[0, :n] = 1
        heads = max(len(tasks), 1)
        options = max(max(len(t.labels) for t in tasks), 1)
        marker_idx = np.zeros((1, heads, options), dtype=np.int32)
        marker_mask = np.zeros((1, heads, options), dtype=np.float32)
        for h, positions in enumerate(markers):
            for o, p in enumerate(positions[:options]):
                marker_idx[0, h, o] = p
                marker_mask[0, h, o] = 1
        return DecisionInput(input_ids, mask, marker_idx, marker_mask)


def tasks_from_json(obj) -> list:
    """`DecisionSchema` (`{"tasks": [...]}`) or a bare task list."""
    items = obj.get("tasks") if isinstance(obj, dict) else obj
    if not isinstance(items, list):
        raise ValueError("a decision schema is {\"tasks\": [...]}")
    return [DecisionTask.from_json(t) for t in items]
