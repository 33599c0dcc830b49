"""Seeded synthetic weights and inputs for the benchmark workloads.

No checkpoint, tokenizer or dataset is available, so every workload is
generated from numpy `default_rng` streams (fp32 draws cast to fp16).  Each
tensor has its own stream keyed by (seed, crc32(name)), so any subset of the
weights (one layer, say) reproduces exactly the values of the full set.

Workloads
  layer        one encoder layer, B=1, L=32, all-ones mask, hidden ~ N(0, 1)
  residual_ln  residual-add LayerNorm, 8192 x 1024: x, res ~ N(0,1),
               gamma ~ N(1, 0.1), beta ~ N(0, 0.1)
  relbias      relative bias + masked softmax, B=32, H=16, L=256, D=64:
               Q, K ~ N(0,1); rel key/query tables [512, 1024] ~ N(0,1);
               valid lengths uniform in [16, 256]
  classify     24-layer encoder + classifier, B=32, L=256, lengths U[40,256],
               ids U[1000, vocab), [CLS] 1 at 0, five [L] markers at 1..5,
               [SEP] 2 at len-1, right-padded with 0
  bucket_mix   4096 rows, lengths log-uniform in [8, 512], smallest bucket of
               L32..L512, 1-2 tasks x 2-10 labels, batches of 32 per bucket
  long_context B=64, L=512 full rows, 3 heads (20, 20, 8 labels), 4-12
               description tokens per label
Weights: linear weights and biases, word and relative embeddings ~ N(0, 0.02);
LayerNorm gamma = 1 + N(0, 0.02), beta ~ N(0, 0.02) (unspecified by the
workload definitions; gamma ~ 1 keeps the hidden states O(1)).
"""

from __future__ import annotations

import zlib
from dataclasses import dataclass

import numpy as np

from .config import DeBERTaV2Configuration
from .decode import DEFAULT_BUCKETS, make_batch_chunk, select_bucket

PAD_ID = 0
CLS_ID = 1
SEP_ID = 2
PROMPT_MARKER_ID = 128001  # "[P]"
LABEL_MARKER_ID = 128002  # "[L]"
SEP_TEXT_ID = 128003
SEP_STRUCT_ID = 128004
OPEN_ID = 1010  # "(" -- ordinary vocabulary ids
CLOSE_ID = 1011  # ")"


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def normal16(seed: int, name: str, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    r = _rng(seed, name)
    x = r.standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    if mean != 0.0:
        x += np.float32(mean)
    return x.astype(np.float16)


def weight_shapes(config: DeBERTaV2Configuration, layers=None) -> dict:
    C, F, V, CH = config.hidden_size, config.intermediate_size, config.vocab_size, config.classifier_hidden
    shapes = {
        "encoder.embeddings.word_embeddings.weight": (V, C),
        "encoder.embeddings.LayerNorm.weight": (C,),
        "encoder.embeddings.LayerNorm.bias": (C,),
        "encoder.encoder.rel_embeddings.weight": (2 * config.position_buckets, C),
        "encoder.encoder.LayerNorm.weight": (C,),
        "encoder.encoder.LayerNorm.bias": (C,),
    }
    idx = range(config.num_hidden_layers) if layers is None else layers
    for i in idx:
        p = f"encoder.encoder.layer.{i}"
        for n in ("query", "key", "value"):
            shapes[f"{p}.attention.self.{n}_proj.weight"] = (C, C)
            shapes[f"{p}.attention.self.{n}_proj.bias"] = (C,)
        shapes[f"{p}.attention.output.dense.weight"] = (C, C)
        shapes[f"{p}.attention.output.dense.bias"] = (C,)
        shapes[f"{p}.attention.output.LayerNorm.weight"] = (C,)
        shapes[f"{p}.attention.output.LayerNorm.bias"] = (C,)
        shapes[f"{p}.intermediate.dense.weight"] = (F, C)
        shapes[f"{p}.intermediate.dense.bias"] = (F,)
        shapes[f"{p}.output.dense.weight"] = (C, F)
        shapes[f"{p}.output.dense.bias"] = (C,)
        shapes[f"{p}.output.LayerNorm.weight"] = (C,)
        shapes[f"{p}.output.LayerNorm.bias"] = (C,)
    shapes["classifier.0.weight"] = (CH, C)
    shapes["classifier.0.bias"] = (CH,)
    shapes["classifier.2.weight"] = (1, CH)
    shapes["classifier.2.bias"] = (1,)
    return shapes


def synthetic_weights(config: DeBERTaV2Configuration, seed: int = 4, layers=None, std: float = 0.02) -> dict:
    """Random-init fp16 weights with the checkpoint key names."""
    out = {}
    for key, shape in weight_shapes(config, layers).items():
        if "LayerNorm.weight" in key:
            out[key] = normal16(seed, key, shape, mean=1.0, std=std)
        else:
            out[key] = normal16(seed, key, shape, std=std)
    return out


# ---------------------------------------------------------------------------
# Standalone-kernel workloads
# ---------------------------------------------------------------------------
def residual_ln_inputs(seed: int = 2, rows: int = 8192, cols: int = 1024):
    return dict(x=normal16(seed, "x", (rows, cols)), residual=normal16(seed, "residual", (rows, cols)),
                gamma=normal16(seed, "gamma", (cols,), 1.0, 0.1), beta=normal16(seed, "beta", (cols,), 0.0, 0.1))


def relbias_inputs(seed: int = 3, batch: int = 32, heads: int = 16, seq_len: int = 256, head_dim: int = 64,
                   positions: int = 512, min_len: int = 16):
    """Q, K [B, H, L, D]; tables [P, H*D]; attention mask [B, L] from lengths."""
    r = _rng(seed, "lengths")
    lengths = r.integers(min_len, seq_len + 1, size=batch)
    mask = (np.arange(seq_len)[None, :] < lengths[:, None]).astype(np.float16)
    return dict(q=normal16(seed, "q", (batch, heads, seq_len, head_dim)),
                k=normal16(seed, "k", (batch, heads, seq_len, head_dim)),
                pos_key=normal16(seed, "pos_key", (positions, heads * head_dim)),
                pos_query=normal16(seed, "pos_query", (positions, heads * head_dim)),
                lengths=lengths, mask=mask)


def layer_inputs(seed: int = 1, batch: int = 1, seq_len: int = 32, hidden: int = 1024):
    return dict(hidden=normal16(seed, "hidden", (batch, seq_len, hidden)),
                mask=np.ones((batch, seq_len), np.float16))


# ---------------------------------------------------------------------------
# Classification workloads
# ---------------------------------------------------------------------------
@dataclass
class Batch:
    input_ids: np.ndarray  # [B, L] int32
    attention_mask: np.ndarray  # [B, L] fp16
    marker_indices: np.ndarray  # [B, Hh, O] int32
    marker_mask: np.ndarray  # [B, Hh, O] fp32
    tasks: list  # per row: list of (num_labels, multi_label)
    valid_rows: int

    @property
    def shape(self):
        B, L = self.input_ids.shape
        return B, L, self.marker_indices.shape[1], self.marker_indices.shape[2]

    def arrays(self) -> dict:
        return dict(input_ids=self.input_ids, attention_mask=self.attention_mask,
                    marker_indices=self.marker_indices, marker_mask=self.marker_mask)


def _schema_row(r: np.random.Generator, task_labels, desc_range, vocab):
    """[CLS] then per task `( [P] prompt ( [L] label desc.. ... ) )` separated
    by [SEP_STRUCT], then [SEP_TEXT] (the layout of NativeTokenizer.swift:
    90-133).  Returns token ids and marker positions per task."""
    ids = [CLS_ID]
    markers = []
    for ti, n in enumerate(task_labels):
        if ti:
            ids.append(SEP_STRUCT_ID)
        ids += [OPEN_ID, PROMPT_MARKER_ID]
        ids += list(r.integers(1000, vocab, size=2))
        ids.append(OPEN_ID)
        pos = []
        for _ in range(n):
            pos.append(len(ids))
            ids.append(LABEL_MARKER_ID)
            nd = int(r.integers(desc_range[0], desc_range[1] + 1)) if desc_range else 1
            ids += list(r.integers(1000, vocab, size=nd))
        ids += [CLOSE_ID, CLOSE_ID]
        markers.append(pos)
    ids.append(SEP_TEXT_ID)
    return ids, markers


def _pack(rows, seq_len: int, max_heads: int, max_options: int) -> tuple:
    B = len(rows)
    ids = np.zeros((B, seq_len), np.int32)
    mask = np.zeros((B, seq_len), np.float16)
    mi = np.zeros((B, max_heads, max_options), np.int32)
    mm = np.zeros((B, max_heads, max_options), np.float32)
    for b, (toks, markers) in enumerate(rows):
        n = len(toks)
        ids[b, :n] = toks
        mask[b, :n] = 1
        for h, pos in enumerate(markers):
            for o, p in enumerate(pos[:max_options]):
                mi[b, h, o] = p
                mm[b, h, o] = 1
    return ids, mask, mi, mm


def classification_batch(seed: int = 4, batch: int = 32, seq_len: int = 256, vocab: int = 128100,
                         num_labels: int = 5, min_len: int = 40) -> Batch:
    """The 24-layer encoder + classifier workload (B=32, L=256, one task of 5
    labels; markers at 1..5)."""
    r = _rng(seed, "classify")
    lengths = r.integers(min_len, seq_len + 1, size=batch)
    rows = []
    for b in range(batch):
        n = int(lengths[b])
        toks = list(r.integers(1000, vocab, size=n))
        toks[0] = CLS_ID
        for j in range(num_labels):
            toks[1 + j] = LABEL_MARKER_ID
        toks[n - 1] = SEP_ID
        rows.append((toks, [list(range(1, 1 + num_labels))]))
    ids, mask, mi, mm = _pack(rows, seq_len, 1, num_labels)
    return Batch(ids, mask, mi, mm, [[(num_labels, False)]] * batch, batch)


def long_context_batch(seed: int = 6, batch: int = 64, seq_len: int = 512, vocab: int = 128100,
                       labels=(20, 20, 8), desc_range=(4, 12)) -> Batch:
    """B=64, L=512, all rows full; heads of 20 and 20 labels (multi-label,
    sigmoid >= 0.5) and 8 labels (single-label).  Description lengths are
    drawn uniformly in [4, 12]; a row whose schema would leave fewer than 16
    text tokens redraws its description lengths from [4, 8]."""
    r = _rng(seed, "long_context")
    rows = []
    for _ in range(batch):
        toks, markers = _schema_row(r, labels, desc_range, vocab)
        if len(toks) > seq_len - 16:
            toks, markers = _schema_row(r, labels, (desc_range[0], 8), vocab)
        toks += list(r.integers(1000, vocab, size=seq_len - len(toks)))
        toks[-1] = SEP_ID
        rows.append((toks[:seq_len], markers))
    ids, mask, mi, mm = _pack(rows, seq_len, len(labels), max(labels))
    tasks = [[(20, True), (20, True), (8, False)]] * batch
    return Batch(ids, mask, mi, mm, tasks, batch)


def bucket_mix(seed: int = 5, count: int = 4096, batch: int = 32, vocab: int = 128100, buckets=DEFAULT_BUCKETS,
               min_len: int = 8, max_len: int = 512) -> list:
    """4096 rows with lengths exp(U(ln 8, ln 512)); each row has 1-2
    single-label tasks of 2-10 labels.  A row whose schema is longer than its
    drawn length is lengthened to fit.  Rows are routed to the smallest
    bucket, then cut into batches of `batch` per bucket, the last batch padded
    with copies of its last row (main.swift:22-49).  Returns a list of Batch."""
    r = _rng(seed, "bucket_mix")
    lengths = np.exp(r.uniform(np.log(min_len), np.log(max_len), size=count))
    lengths = np.clip(np.round(lengths).astype(int), min_len, max_len)
    per_bucket: dict = {}
    for i in range(count):
        nt = int(r.integers(1, 3))
        labels = [int(r.integers(2, 11)) for _ in range(nt)]
        toks, markers = _schema_row(r, labels, None, vocab)
        n = max(int(lengths[i]), len(toks) + 1)
        n = min(n, max_len)
        toks += list(r.integers(1000, vocab, size=max(0, n - len(toks))))
        toks = toks[:n]
        toks[-1] = SEP_ID
        per_bucket.setdefault(select_bucket(n, buckets), []).append((toks, markers, [(k, False) for k in labels]))
    out = []
    for L in sorted(per_bucket):
        rows = per_bucket[L]
        for s in range(0, len(rows), batch):
            chunk = rows[s:s + batch]
            hh = max(len(m) for _, m, _ in chunk)
            oo = max(max(len(p) for p in m) for _, m, _ in chunk)
            ids, mask, mi, mm = _pack([(t, m) for t, m, _ in chunk], L, hh, oo)
            arrays, valid = make_batch_chunk(dict(input_ids=ids, attention_mask=mask, marker_indices=mi,
                                                  marker_mask=mm), 0, len(chunk), batch)
            tasks = [tk for _, _, tk in chunk]
            tasks += [tasks[-1]] * (batch - len(chunk))
            out.append(Batch(arrays["input_ids"], arrays["attention_mask"], arrays["marker_indices"],
                             arrays["marker_mask"], tasks, valid))
    return out


# Text workload of the JSONL runner: a word-level tokenizer over synthetic
# words (every word one token, as in the id-level workloads above) and
# examples whose total token counts follow the bucket mix.
SERVING_WORDS = 60000


def word_level_frontend(words: int = SERVING_WORDS):
    """NativeDecisionTokenizer (the C++ front end) over a word-level
    vocabulary: the reference's
    added tokens ([PAD] 0, [CLS] 1, [SEP] 2, [UNK] 3, [MASK] 4, [P], [L],
    [SEP_TEXT], [SEP_STRUCT], [DESCRIPTION] at 128001..128005), punctuation,
    task and label names, and `words` synthetic words w0, w1, ... from id
    2000 on."""
    import json
    from .frontend import NativeDecisionTokenizer
    return NativeDecisionTokenizer.from_json(json.dumps(word_level_tokenizer_json(words)))


def word_level_tokenizer_json(words: int = SERVING_WORDS) -> dict:
    """The tokenizer.json of word_level_frontend: a WordLevel model behind a
    WhitespaceSplit pre-tokenizer, the specials as added tokens."""
    specials = {"[PAD]": PAD_ID, "[CLS]": CLS_ID, "[SEP]": SEP_ID, "[UNK]": 3, "[MASK]": 4,
                "[P]": PROMPT_MARKER_ID, "[L]": LABEL_MARKER_ID, "[SEP_TEXT]": SEP_TEXT_ID,
                "[SEP_STRUCT]": SEP_STRUCT_ID, "[DESCRIPTION]": 128005}
    vocab = dict(specials)
    vocab.update({"(": OPEN_ID, ")": CLOSE_ID, ".": 1012, ":": 1013})
    vocab.update({f"task{i}": 1100 + i for i in range(8)})
    vocab.update({f"l{i}": 1200 + i for i in range(32)})
    vocab.update({f"w{i}": 2000 + i for i in range(words)})
    added = [{"id": i, "content": t, "single_word": False, "lstrip": False, "rstrip": False, "normalized": False,
              "special": True} for t, i in specials.items()]
    return {"version": "1.0", "truncation": None, "padding": None, "added_tokens": added, "normalizer": None,
            "pre_tokenizer": {"type": "WhitespaceSplit"}, "post_processor": None, "decoder": None,
            "model": {"type": "WordLevel", "vocab": vocab, "unk_token": "[UNK]"}}


def serving_examples(seed: int = 7, count: int = 4096, words: int = SERVING_WORDS, min_len: int = 8,
                     max_len: int = 512) -> list:
    """JSONL example objects {"id", "text", "tasks"}: 1-2 single-label tasks
    of 2-10 labels, total token counts exp(U(ln 8, ln 512)) (schema + text +
    the final "."; at least one text word), text words drawn Zipf(1.1) over
    the synthetic vocabulary."""
    r = _rng(seed, "serving")
    lengths = np.exp(r.uniform(np.log(min_len), np.log(max_len), size=count))
    out = []
    for i in range(count):
        labels = [int(r.integers(2, 11)) for _ in range(int(r.integers(1, 3)))]
        tasks = [{"name": f"task{t}", "labels": [f"l{j}" for j in range(n)], "multiLabel": False}
                 for t, n in enumerate(labels)]
        schema = sum(6 + 2 * n for n in labels) + len(labels)  # groups, [SEP_STRUCT]s, [SEP_TEXT]
        n_words = int(min(max(1, round(lengths[i]) - schema - 1), max_len - schema - 1))
        ranks = np.minimum(r.zipf(1.1, size=n_words), words) - 1
        out.append({"id": f"s{i}", "text": " ".join(f"w{k}" for k in ranks), "tasks": tasks})
    return out
