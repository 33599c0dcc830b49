"""Schema formatter and tokenizer front end: `NativeDecisionTokenizer`
(NativeTokenizer.swift:56-212).

Two backends with the same behaviour:
* "native" (the default for a tokenizer directory): the C++ front end of
  libgliner_decide_frontend.so -- ICU's regular expressions for the word
  split (the engine behind NSRegularExpression) and a C++ restatement of the
  tokenizer.json pipeline (normaliser, Metaspace pre-tokenizer, Unigram
  Viterbi);
* "hf": the same steps in Python over the HF `tokenizers` library
  (`tokenizers.Tokenizer.encode(..., add_special_tokens=False)`), used for an
  in-memory `tokenizers.Tokenizer` and as the check of the native backend.

The steps (both backends):

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
# case-insensitive, restated for the `regex` module without its IGNORECASE
# (whose folding also lets U+0130 match [a-z], which ICU's does not):
# * ICU's \w = [\p{Alphabetic}\p{Mark}\p{Decimal_Number}
#   \p{Connector_Punctuation}\u200c\u200d] (Python's \w has no combining
#   marks) and \s = [\t\n\f\r\p{Z}]; both are closed under case already;
# * a case-insensitive [a-z] is ICU's case closure of it, A-Z a-z plus U+017F
#   (long s) and U+212A (Kelvin sign); the literal letters of "https" and "www"
#   match their closures the same way.
_W = r"[\p{Alphabetic}\p{M}\p{Nd}\p{Pc}\u200c\u200d]"
_NS = r"[^\t\n\f\r\p{Z}]"
_AZ = "A-Za-z\u017f\u212a"
WORD_PATTERN = regex.compile(
    rf"(?:[hH][tT][tT][pP][sS\u017f]?://{_NS}+|[wW][wW][wW]\.{_NS}+)|[{_AZ}0-9._%+-]+@[{_AZ}0-9.-]+\.[{_AZ}]{{2,}}"
    rf"|@[{_AZ}0-9_]+|{_W}+(?:[-_]{_W}+)*|{_NS}",
    regex.V0)


class TokenizerError(ValueError):
    """NativeTokenizerError (NativeTokenizer.swift:5-23)."""


def _lower_scalars(word: str) -> str:
    # Swift's String.lowercased(): each scalar's full lower-case mapping, with
    # no context (a final capital sigma becomes the plain small sigma).
    return "".join(ch.lower() for ch in word)


_PREPEND = regex.compile(r"\p{Grapheme_Cluster_Break=Prepend}")


def _ends_sentence(text: str) -> bool:
    # Swift's `text.last` is the last grapheme cluster: a final '.', '!' or
    # '?' stands alone unless a Prepend character before it joins it.
    return text[-1] in ".!?" and not (len(text) > 1 and _PREPEND.match(text[-2]))


def split_words(text: str) -> list:
    """NativeTokenizer.swift:193-208."""
    if not text:
        normalized = "."
    elif _ends_sentence(text):
        normalized = text
    else:
        normalized = text + "."
    return [_lower_scalars(w) for w in WORD_PATTERN.findall(normalized)]


def load_added_tokens(tokenizer_json: str | Path) -> dict:
    """`added_tokens` content -> id of a tokenizer.json (NativeTokenizer.swift:210-226)."""
    root = json.loads(Path(tokenizer_json).read_text(encoding="utf-8"))
    out = {}
    for tok in root.get("added_tokens") or []:
        content, tid = tok.get("content"), tok.get("id")
        if isinstance(content, str) and isinstance(tid, int):
            out[content] = tid
    return out


class _NativeFrontend:
    """A gd_frontend handle (include/gliner_decide_frontend.h)."""

    def __init__(self, directory=None, tokenizer_json: str | None = None):
        import ctypes as C
        from . import _frontend_native as F
        self._C, self._F = C, F
        self._lib = F.lib()
        h = C.c_void_p()
        try:
            if directory is not None:
                F.check(self._lib.gd_frontend_open(C.byref(h), str(directory).encode()))
            else:
                b = tokenizer_json.encode("utf-8")
                F.check(self._lib.gd_frontend_create(C.byref(h), b, len(b)))
        except F.FrontendError as e:
            raise TokenizerError(str(e)) from e
        self._h = h
        pad = C.c_int32()
        F.check(self._lib.gd_frontend_pad_id(h, C.byref(pad)))
        self.pad_token_id = int(pad.value)

    def _call(self, fn, *args):
        try:
            self._F.check(fn(self._h, *args))
        except self._F.FrontendError as e:
            raise TokenizerError(str(e)) from e

    def _ids(self, fn, text: str) -> list:
        C = self._C
        b = text.encode("utf-8")
        cap = 2 * len(b) + 16  # enough unless normalisation expands the text; then the size reported
        for _ in range(2):
            buf = (C.c_int32 * cap)()
            n = C.c_int64()
            status = fn(self._h, b, len(b), buf, cap, C.byref(n))
            if status == self._F.GD_ERR_SHAPE and n.value > cap:
                cap = n.value
                continue
            self._call(lambda h: status)
            return list(buf[:n.value])
        raise TokenizerError("token count changed between two calls")

    def encode(self, text: str) -> list:
        return self._ids(self._lib.gd_frontend_encode, text)

    def append_tokenized(self, text: str, ids: list) -> None:
        ids.extend(self._ids(self._lib.gd_frontend_append_tokenized, text))

    def split_words(self, text: str) -> list:
        C = self._C
        b = text.encode("utf-8")
        cap = 4 * len(b) + 16  # a word's lower case is at most 3x its bytes, plus its NUL and the final '.'
        buf = C.create_string_buffer(cap)
        nb, nw = C.c_int64(), C.c_int64()
        self._call(self._lib.gd_frontend_split_words, b, len(b), buf, cap, C.byref(nb), C.byref(nw))
        raw = buf.raw[:nb.value]
        return [w.decode("utf-8") for w in raw.split(b"\0")[:nw.value]]

    def clear_cache(self) -> None:
        self._call(self._lib.gd_frontend_clear_cache)

    def make_arrays(self, text: str, tasks, buckets):
        """(input_ids [L], mask [L] fp16, markers [Hh*O], marker mask, L, n, Hh, O)."""
        C = self._C
        tb = text.encode("utf-8")
        sj = json.dumps([t.to_json() for t in tasks], ensure_ascii=False).encode("utf-8")
        bl = [int(b) for b in buckets]
        barr = (C.c_int64 * max(len(bl), 1))(*bl)
        cap = max([b for b in bl if b > 0], default=0)
        heads = max(len(tasks), 1)
        options = max([len(t.labels) for t in tasks], default=1) or 1
        ids = np.zeros(max(cap, 1), np.int32)
        mask = np.zeros(max(cap, 1), np.float16)
        mi = np.zeros(heads * options, np.int32)
        mm = np.zeros(heads * options, np.float32)
        L, n, hh, oo = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64()
        self._call(self._lib.gd_frontend_make_input, tb, len(tb), sj, len(sj), barr, len(bl),
                   ids.ctypes.data_as(C.POINTER(C.c_int32)), mask.ctypes.data_as(C.POINTER(C.c_uint16)), ids.size,
                   mi.ctypes.data_as(C.POINTER(C.c_int32)), mm.ctypes.data_as(C.POINTER(C.c_float)), mi.size,
                   C.byref(L), C.byref(n), C.byref(hh), C.byref(oo))
        return ids[:L.value], mask[:L.value], mi, mm, L.value, n.value, hh.value, oo.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.gd_frontend_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class NativeDecisionTokenizer:
    """Mirror of `NativeDecisionTokenizer` (NativeTokenizer.swift:56-75).

    `NativeDecisionTokenizer(directory)` reads tokenizer.json (and requires
    tokenizer_config.json beside it, as the reference does) into the C++
    front end (`backend="hf"` runs the HF `tokenizers` library instead);
    `from_tokenizer(tokenizer, special_ids)` wraps a `tokenizers.Tokenizer`
    built in memory (HF backend, or the C++ one from its JSON with
    `backend="native"`, whose added tokens are then the special ids)."""

    def __init__(self, directory: str | Path | None = None, *, tokenizer=None, special_ids: dict | None = None,
                 backend: str | None = None):
        if backend not in (None, "native", "hf"):
            raise ValueError(f"backend must be 'native' or 'hf' (got {backend!r})")
        self.backend = backend or ("native" if directory is not None else "hf")
        self._native = None
        self._tokenizer_json = None
        if self.backend == "native":
            if directory is not None:
                self._native = _NativeFrontend(directory=directory)
                self._tokenizer_json = Path(directory) / "tokenizer.json"
            else:
                if tokenizer is None:
                    raise TokenizerError("a tokenizer directory or a tokenizers.Tokenizer is required")
                text = tokenizer.to_str()
                self._native = _NativeFrontend(tokenizer_json=text)
                self._special = {t["content"]: t["id"] for t in json.loads(text).get("added_tokens") or []}
                if special_ids is not None and dict(special_ids) != self._special:
                    raise TokenizerError("with the native backend the special ids are the tokenizer's added tokens")
            self.tokenizer = tokenizer
            self.pad_token_id = self._native.pad_token_id
            return
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
    def from_tokenizer(cls, tokenizer, special_ids: dict | None = None,
                       backend: str = "hf") -> "NativeDecisionTokenizer":
        return cls(tokenizer=tokenizer, special_ids=special_ids, backend=backend)

    @classmethod
    def from_json(cls, tokenizer_json: str, backend: str = "native") -> "NativeDecisionTokenizer":
        """From tokenizer.json text; the special ids are its added tokens."""
        special = {t["content"]: t["id"] for t in json.loads(tokenizer_json).get("added_tokens") or []}
        if backend == "hf":
            from tokenizers import Tokenizer
            return cls(tokenizer=Tokenizer.from_str(tokenizer_json), special_ids=special, backend="hf")
        self = cls.__new__(cls)
        self.backend = "native"
        self.tokenizer = None
        self._tokenizer_json = None
        self._native = _NativeFrontend(tokenizer_json=tokenizer_json)
        self._special = special
        self.pad_token_id = self._native.pad_token_id
        return self

    @property
    def special_ids(self) -> dict:
        if self._native is None:
            return self._special_ids
        if not hasattr(self, "_special"):
            self._special = load_added_tokens(self._tokenizer_json)
        return self._special

    @special_ids.setter
    def special_ids(self, value: dict) -> None:
        self._special_ids = value

    def clear_cache(self) -> None:
        """Empties the entry cache (ids of recent schema entries and words)."""
        if self._native is not None:
            self._native.clear_cache()
        else:
            self._cache.clear()

    def split_words(self, text: str) -> list:
        return self._native.split_words(text) if self._native is not None else split_words(text)

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
        if self._native is not None:
            self._native.append_tokenized(text, ids)
            return
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
        if self._native is not None:
            tasks = list(tasks)
            ids, _, mi, mm, _, n, hh, oo = self._native.make_arrays(text, tasks, [1 << 20])
            mi, mm = mi.reshape(hh, oo), mm.reshape(hh, oo)
            return [int(x) for x in ids[:n]], [[int(p) for p, m in zip(mi[t], mm[t]) if m > 0]
                                              for t in range(len(tasks))]
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
        if self._native is not None:
            ids, mask, mi, mm, L, _, hh, oo = self._native.make_arrays(text, tasks, buckets)
            return DecisionInput(ids.reshape(1, L).copy(), mask.reshape(1, L).copy(), mi.reshape(1, hh, oo),
                                 mm.reshape(1, hh, oo))
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
