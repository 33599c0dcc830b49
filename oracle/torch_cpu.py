"""fp32 torch-CPU restatement of the default reference graph: the CPU baseline.

TEST INFRASTRUCTURE ONLY.  Run by the `cpu_baseline` leg of `bench.py` (and
pinned by `tests/test_oracle.py`); never by the product path.

The reference has no CPU switch and its Metal kernels cannot run on a CPU;
this is the same graph as `oracle.deberta.OracleModel` (default flags:
DeBERTa.swift:274-447 with the relative bias of :374-379 and SDPA of
:382-395), batched over the rows and evaluated in float32 without the fp16
rounding points, with torch's multithreaded CPU kernels -- the fastest
faithful CPU evaluation available in this environment.  Every row is
computed at the full bucket length L, as the reference does.

With round16=True the same graph rounds to fp16 wherever the reference
writes an fp16 array (the rounding points of `oracle.deberta`: every addMM
output, c2pRaw / p2cRaw, their sum and its division by fp16(sqrt(3D)), the
bias + key-mask add, the attention output, the residual sums, LayerNorm and
GELU outputs, the classifier's logits) and evaluates between them in fp32:
a second restatement of the GPU's rounding chain, fast enough to check whole
batches at the label-probability bar.  It is pinned against the numpy
oracle (float64 and float32, same rounding points) in tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np
import torch

from . import deberta as O


def _t(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32)))


class TorchCPUModel:
    """`GLiNERDecideClassifier` (default flags) on torch CPU tensors, fp32."""

    def __init__(self, weights: dict, config: O.Config, round16: bool = False):
        self.c = config
        self.round16 = round16
        r = self._r
        C, H = config.hidden_size, config.num_attention_heads
        self.H, self.D = H, C // H
        w = O.ModelWeights.from_store(weights, config)
        self.emb = _t(w.word_embeddings)
        self.emb_g, self.emb_b = _t(w.emb_ln_g), _t(w.emb_ln_b)
        self.layers = []
        eps = config.layer_norm_eps
        # relative precompute (DeBERTa.swift:204-227)
        rel_n = r(torch.nn.functional.layer_norm(_t(w.rel_embeddings), (C,), _t(w.rel_ln_g), _t(w.rel_ln_b), eps))
        for lw in w.layers:
            qkv_w, qkv_b = _t(lw.qkv_w), _t(lw.qkv_b)
            pos = r(rel_n @ qkv_w[: 2 * C].T + qkv_b[: 2 * C]).view(O.POSITION_COUNT, 2, H, self.D)
            self.layers.append(dict(
                qkv_w=qkv_w, qkv_b=qkv_b, pos_q=pos[:, 0].permute(1, 0, 2).contiguous(),
                pos_k=pos[:, 1].permute(1, 0, 2).contiguous(), out_w=_t(lw.out_w), out_b=_t(lw.out_b),
                ln1_g=_t(lw.ln1_g), ln1_b=_t(lw.ln1_b), inter_w=_t(lw.inter_w), inter_b=_t(lw.inter_b),
                ffn_w=_t(lw.ffn_out_w), ffn_b=_t(lw.ffn_out_b), ln2_g=_t(lw.ln2_g), ln2_b=_t(lw.ln2_b)))
        self.cls0_w, self.cls0_b = _t(w.cls0_w), _t(w.cls0_b)
        self.cls2_w, self.cls2_b = _t(w.cls2_w), _t(w.cls2_b)
        self._idx = {}

    def _r(self, t: torch.Tensor) -> torch.Tensor:
        """An fp16 rounding point (identity unless round16)."""
        return t.half().float() if self.round16 else t

    def _indices(self, L: int):
        if L not in self._idx:
            c2p, p2c = O.relative_indices(L, self.c.position_buckets)
            self._idx[L] = (torch.from_numpy(c2p), torch.from_numpy(p2c))
        return self._idx[L]

    @torch.no_grad()
    def forward(self, ids, attention_mask, marker_indices, marker_mask) -> torch.Tensor:
        """Logits [B, Hh, O] (fp32) for host arrays of one batch."""
        r = self._r
        x = self.encode(ids, attention_mask)
        B, L, C = x.shape
        mi = torch.from_numpy(np.asarray(marker_indices, np.int64))  # :430-444
        flat = (mi + (torch.arange(B) * L)[:, None, None]).reshape(-1)
        m = x.reshape(B * L, C)[flat]
        val = r(torch.relu(r(m @ self.cls0_w.T + self.cls0_b)) @ self.cls2_w.T + self.cls2_b)[:, 0].view(mi.shape)
        mm = _t(marker_mask)
        return r(torch.where(mm > 0, val, torch.tensor(O.LOGIT_FILL)))

    @torch.no_grad()
    def encode(self, ids, attention_mask) -> torch.Tensor:
        """Final hidden states [B, L, C] (fp32) for host arrays of one batch."""
        c, H, D = self.c, self.H, self.D
        C, eps = c.hidden_size, c.layer_norm_eps
        r = self._r
        ids = torch.from_numpy(np.asarray(ids, np.int64))
        mask = _t(attention_mask)
        B, L = ids.shape
        ln = torch.nn.functional.layer_norm
        x = r(r(ln(self.emb[ids], (C,), self.emb_g, self.emb_b, eps)) * mask[..., None])  # :285-292
        c2p_idx, p2c_idx = self._indices(L)
        ci = c2p_idx.expand(B, H, L, L)
        pi = p2c_idx.expand(B, H, L, L)
        key_mask = torch.where(mask > 0, 0.0, O.MASK_FILL)[:, None, None, :]  # :329-335
        bias_scale = O.scale_f16(D)  # fp16(sqrt(3D)) (:323-326)
        qk_scale = O.scale_f32(D)  # 1 / sqrt(3D) (:390)
        for p in self.layers:
            qkv = r(x @ p["qkv_w"].T + p["qkv_b"]).view(B, L, 3, H, D)  # :298-320
            q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
            c2p = torch.gather(r(q @ p["pos_k"].transpose(-1, -2)), -1, ci)  # :374-375
            p2c = torch.gather(r(k @ p["pos_q"].transpose(-1, -2)), -1, pi).transpose(-1, -2)  # :376-378
            bias = r(r(c2p + p2c) / bias_scale)  # :379
            del c2p, p2c
            scores = q @ k.transpose(-1, -2) * qk_scale + r(bias + key_mask)  # :383-392
            del bias
            ctx = r((torch.softmax(scores, -1) @ v).permute(0, 2, 1, 3).reshape(B, L, C))
            del scores
            x = r(ln(r(r(ctx @ p["out_w"].T + p["out_b"]) + x), (C,), p["ln1_g"], p["ln1_b"], eps))  # :412-418
            inter = r(torch.nn.functional.gelu(r(x @ p["inter_w"].T + p["inter_b"])))  # :420-421
            x = r(ln(r(r(inter @ p["ffn_w"].T + p["ffn_b"]) + x), (C,), p["ln2_g"], p["ln2_b"], eps))  # :422-427
        return x

    @staticmethod
    def flops(B: int, L: int, config: O.Config) -> float:
        """Dense FLOPs of one forward (linear layers, relative projections,
        attention products), for the rate's context."""
        C, F, N = config.hidden_size, config.intermediate_size, config.num_hidden_layers
        per_layer = 2 * B * L * C * (3 * C + C + 2 * F) + 2 * B * L * O.POSITION_COUNT * C * 2 + 4 * B * L * L * C
        return float(N * per_layer)


def cpu_description() -> str:
    """CPU model name of this host (from /proc/cpuinfo), for the report."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"

