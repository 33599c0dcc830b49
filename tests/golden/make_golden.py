"""Writes the golden fixtures under tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

Sources, all independent of `oracle/`:
  * HF transformers DeBERTa-v2 (`make_log_bucket_position`, `DebertaV2Model`)
    -- a third-party implementation of the same architecture, used in float64
    on the CPU with weights built from a local config (nothing downloaded);
  * brute-force scalar loops over the reference's own known-answer generators
    (main.swift:141-192), written here element by element;
  * closed forms (main.swift:194-225 LayerNorm known answer).
The fixtures are data (inputs and expected outputs); the tests compare the
oracle and the HIP path against them.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "gliner-decide-metal_amd"))


def hf_bucket_table():
    """idx(r) = clip(bucket(r) + 256, 0, 511) from HF make_log_bucket_position,
    r in [-511, 511]."""
    import torch
    from transformers.models.deberta_v2.modeling_deberta_v2 import make_log_bucket_position

    r = torch.arange(-511, 512, dtype=torch.long)
    b = make_log_bucket_position(r, 256, 512).to(torch.long).numpy()
    np.save(OUT / "relative_bucket_256_512.npy", b.astype(np.int32))
    print("relative_bucket_256_512.npy", b.min(), b.max())


def f16(x):
    return float(np.float16(x))


def reference_relbias_known_answer():
    """main.swift:141-192 generators, B=1 H=2 L=8 D=4 P=8, general indices
    c2p = i % 8, p2c = 3i % 8, keys >= 6 masked.  Expected values computed
    with explicit loops in float64:
      kernel  (c2p + p2c) * (1/sqrt(12) as fp32)             (FusedKernels)
      graph   fp16(fp16(fp16(c2p) + fp16(p2c)) / fp16(sqrt 12))  (MLX ops)
    plus the fused-attention kernel output with v = (11 i % 29) / 29."""
    b, h, l, d, p = 1, 2, 8, 4, 8
    q = np.array([f16((i % 13) / 13.0) for i in range(b * h * l * d)]).reshape(b, h, l, d)
    k = np.array([f16(((i * 7) % 17) / 17.0) for i in range(b * h * l * d)]).reshape(b, h, l, d)
    v = np.array([f16(((i * 11) % 29) / 29.0) for i in range(b * h * l * d)]).reshape(b, h, l, d)
    pk = np.array([f16(((i * 3) % 19) / 19.0) for i in range(h * p * d)]).reshape(h, p, d)
    pq = np.array([f16(((i * 5) % 23) / 23.0) for i in range(h * p * d)]).reshape(h, p, d)
    c2p = np.array([i % p for i in range(h * l * l)], np.int32).reshape(h, l, l)
    p2c = np.array([(i * 3) % p for i in range(h * l * l)], np.int32).reshape(h, l, l)
    mask = np.array([0.0 if j < 6 else -65504.0 for j in range(l)])
    scale32 = float(np.float32(1.0) / np.float32(math.sqrt(d * 3)))
    scale16 = f16(math.sqrt(d * 3))
    kern = np.zeros((b, h, l, l))
    graph = np.zeros((b, h, l, l))
    fused = np.zeros((b, l, h, d))
    for hh in range(h):
        for qi in range(l):
            scores = []
            for ki in range(l):
                a = sum(q[0, hh, qi, t] * pk[hh, c2p[hh, qi, ki], t] for t in range(d))
                c = sum(k[0, hh, ki, t] * pq[hh, p2c[hh, ki, qi], t] for t in range(d))
                qk = sum(q[0, hh, qi, t] * k[0, hh, ki, t] for t in range(d))
                masked = mask[ki] < -60000.0
                kern[0, hh, qi, ki] = -65504.0 if masked else (a + c) * scale32
                graph[0, hh, qi, ki] = -65504.0 if masked else f16(f16(f16(a) + f16(c)) / scale16)
                scores.append(-65504.0 if masked else (qk + a + c) * scale32)
            m = max(max(scores), -65504.0)
            e = [math.exp(s - m) for s in scores]
            tot = sum(e)
            for t in range(d):
                fused[0, qi, hh, t] = sum(e[ki] / tot * v[0, hh, ki, t] for ki in range(l))
    np.savez(OUT / "relbias_known_answer.npz", q=q, k=k, v=v, pos_key=pk, pos_query=pq, c2p=c2p, p2c=p2c,
             key_mask=mask.reshape(1, l), scale=np.float32(scale32), kernel=kern, graph=graph, fused=fused)
    print("relbias_known_answer.npz")


def ln_known_answer():
    """main.swift:194-225: x_i = i/1024 (exact in fp16), residual 0, gamma 1,
    beta 0, eps 1e-7.  mean = 1023/2048, biased var = (1024^2 - 1)/(12*1024^2)."""
    n = 1024
    x = np.arange(n) / 1024.0
    mean = (n - 1) / (2.0 * n)
    var = (n * n - 1) / (12.0 * n * n)
    y = (x - mean) / math.sqrt(var + 1e-7)
    np.savez(OUT / "ln_known_answer.npz", x=x.astype(np.float16), expected=y)
    print("ln_known_answer.npz")


def hf_model(config_kwargs, weights: dict, ids, mask, layers: int):
    import torch
    from transformers import DebertaV2Config
    from transformers.models.deberta_v2.modeling_deberta_v2 import DebertaV2Model

    cfg = DebertaV2Config(relative_attention=True, position_buckets=256, max_relative_positions=-1,
                          max_position_embeddings=512, pos_att_type=["p2c", "c2p"], share_att_key=True,
                          norm_rel_ebd="layer_norm", layer_norm_eps=1e-7, hidden_act="gelu",
                          position_biased_input=False, type_vocab_size=0, hidden_dropout_prob=0.0,
                          attention_probs_dropout_prob=0.0, num_hidden_layers=layers, **config_kwargs)
    model = DebertaV2Model(cfg).double().eval()
    sd = {}
    for k, v in weights.items():
        if k.startswith("encoder."):
            sd[k[len("encoder."):]] = torch.from_numpy(np.asarray(v, np.float64))
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not [m for m in missing if "position_ids" not in m], missing
    with torch.no_grad():
        out = model(input_ids=torch.from_numpy(ids.astype(np.int64)),
                    attention_mask=torch.from_numpy(mask.astype(np.int64)), output_hidden_states=True)
    return [h.numpy() for h in out.hidden_states]


def hf_fixtures():
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.synthetic import synthetic_weights

    # (1) full width, L = 32, B = 1, all-ones mask, 1 layer (the single-layer workload)
    cfg = DeBERTaV2Configuration(num_hidden_layers=1, vocab_size=2048)
    w = synthetic_weights(cfg, seed=1)
    r = np.random.default_rng(11)
    ids = r.integers(3, 2048, size=(1, 32)).astype(np.int32)
    mask = np.ones((1, 32), np.float16)
    hs = hf_model(dict(hidden_size=1024, num_attention_heads=16, intermediate_size=4096, vocab_size=2048), w, ids,
                  mask, 1)
    np.savez_compressed(OUT / "hf_layer_c1024_l32.npz", ids=ids, mask=mask, embed=hs[0].astype(np.float32),
                        out=hs[1].astype(np.float32))
    print("hf_layer_c1024_l32.npz")

    # (2) narrow model (2 heads of 64), L = 256 so the log buckets are used,
    # 2 layers, padded rows (compare valid rows only).
    cfg = DeBERTaV2Configuration(hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                                 num_attention_heads=2, vocab_size=512, classifier_hidden=256)
    w = synthetic_weights(cfg, seed=7)
    r = np.random.default_rng(12)
    B, L = 2, 256
    ids = r.integers(3, 512, size=(B, L)).astype(np.int32)
    lengths = np.array([256, 173])
    mask = (np.arange(L)[None, :] < lengths[:, None]).astype(np.float16)
    ids[mask == 0] = 0
    hs = hf_model(dict(hidden_size=128, num_attention_heads=2, intermediate_size=256, vocab_size=512), w, ids, mask, 2)
    np.savez_compressed(OUT / "hf_encoder_c128_l256.npz", ids=ids, mask=mask, lengths=lengths,
                        out=hs[2].astype(np.float32), layer1=hs[1].astype(np.float32))
    print("hf_encoder_c128_l256.npz")


if __name__ == "__main__":
    hf_bucket_table()
    reference_relbias_known_answer()
    ln_known_answer()
    hf_fixtures()
