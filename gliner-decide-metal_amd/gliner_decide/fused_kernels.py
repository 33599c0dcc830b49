"""`FusedKernels` (FusedKernels.swift:7-286) on the HIP library.

Same method names and argument meaning as the Swift class; tensors are torch
GPU tensors, outputs are allocated by the callee (as MLX's
`outputShapes`/`outputDTypes`), and shape misuse raises GlinerDecideError
instead of trapping.  The default-graph kernels the encoder runs (fused
relative bias + masked softmax + P.V, embedding LayerNorm, linear epilogues)
are exposed beside them.
"""

from __future__ import annotations

import math

import torch

from . import _native as N
from .device import as_f16, as_i32, ptr, stream_handle


def _dims(t: torch.Tensor, n: int, name: str):
    if t.dim() != n:
        raise N.GlinerDecideError(N.GD_ERR_SHAPE, f"{name} must have {n} dimensions (got {tuple(t.shape)})")
    return tuple(t.shape)


def _indices(c2p_indices, p2c_indices, H: int, L: int):
    """General index tensors broadcast to [H, L, L], or (None, None) for the
    closed form."""
    if c2p_indices is None and p2c_indices is None:
        return None, None
    if c2p_indices is None or p2c_indices is None:
        raise N.GlinerDecideError(N.GD_ERR_INVALID_ARGUMENT, "give both index tensors, or neither")
    c2p = as_i32(c2p_indices, "c2p_indices").expand(1, H, L, L).reshape(H, L, L).contiguous()
    p2c = as_i32(p2c_indices, "p2c_indices").expand(1, H, L, L).reshape(H, L, L).contiguous()
    return c2p, p2c


class FusedKernels:
    """Mirror of `FusedKernels` (FusedKernels.swift:7)."""

    def __init__(self):
        self._lib = N.lib()

    # -- FusedKernels.residualLayerNorm (FusedKernels.swift:261-286) --------
    def residual_layer_norm(self, x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
                            bias: torch.Tensor, eps: float, round_sum_f16: bool = False) -> torch.Tensor:
        """LayerNorm(x + residual) * weight + bias over the last axis.

        round_sum_f16=False keeps x + residual in fp32 (the Metal kernel);
        True rounds it to fp16 first (the default graph `norm(x + residual)`,
        DeBERTa.swift:463).  residual=None gives a plain LayerNorm."""
        x = as_f16(x, "x")
        if residual is not None:
            residual = as_f16(residual, "residual")
            if residual.shape != x.shape:
                raise N.GlinerDecideError(N.GD_ERR_SHAPE, "residual shape mismatch")
        if x.dim() < 1:
            raise N.GlinerDecideError(N.GD_ERR_SHAPE, "x must have at least one dimension")
        cols = x.shape[-1]
        rows = x.numel() // cols if cols else 0
        weight = as_f16(weight, "weight")
        bias = as_f16(bias, "bias")
        out = torch.empty_like(x)
        N.check(self._lib.gd_residual_layer_norm(ptr(x), ptr(residual), ptr(weight), ptr(bias), ptr(out), rows, cols,
                                                 float(eps), N.GD_LN_SUM_F16 if round_sum_f16 else 0,
                                                 stream_handle()))
        return out

    # -- FusedKernels.relativeBias (FusedKernels.swift:214-258) -------------
    def relative_bias(self, q, k, position_key, position_query, c2p_indices, p2c_indices, key_mask, scale: float,
                      batch: int, heads: int, sequence_length: int, head_dimension: int,
                      position_count: int) -> torch.Tensor:
        """(q.posK[c2p] + k.posQ[p2c]) * scale with masked keys := -65504,
        general index tensors [1 or H, L, L]; returns [B, H, L, L] fp16.
        c2p_indices = p2c_indices = None selects the closed-form indices
        (the ones the classifier builds) on the MFMA attention kernel."""
        q = as_f16(q, "q")
        k = as_f16(k, "k")
        if q.shape != k.shape or q.dim() != 4 or q.shape[2] != sequence_length or q.shape[3] != head_dimension:
            raise N.GlinerDecideError(N.GD_ERR_SHAPE, "q/k must both be [B, H, L, D]")
        H, L = heads, sequence_length
        c2p, p2c = _indices(c2p_indices, p2c_indices, H, L)
        pk = as_f16(position_key, "position_key").reshape(H, position_count, head_dimension).contiguous()
        pq = as_f16(position_query, "position_query").reshape(H, position_count, head_dimension).contiguous()
        km = as_f16(key_mask, "key_mask").reshape(batch, L).contiguous()
        out = torch.empty((batch, H, L, L), dtype=torch.float16, device=q.device)
        N.check(self._lib.gd_relative_bias(ptr(q), ptr(k), ptr(pk), ptr(pq), ptr(c2p), ptr(p2c), ptr(km),
                                           float(scale), batch, H, L, head_dimension, position_count, ptr(out),
                                           stream_handle()))
        return out

    # -- FusedKernels.fusedAttention (FusedKernels.swift:160-210) -----------
    def fused_attention(self, queries, keys, values, position_key, position_query, c2p_indices, p2c_indices,
                        key_mask, scale: float, batch: int, heads: int, sequence_length: int, head_dimension: int,
                        position_count: int) -> torch.Tensor:
        """Whole attention with general indices (None for the closed form, on
        the MFMA attention kernel); returns [B, L, H, D] fp16."""
        q = as_f16(queries, "queries")
        k = as_f16(keys, "keys")
        v = as_f16(values, "values")
        if not (q.shape == k.shape == v.shape) or q.dim() != 4:
            raise N.GlinerDecideError(N.GD_ERR_SHAPE, "queries/keys/values must all be [B, H, L, D]")
        if tuple(q.shape) != (batch, heads, sequence_length, head_dimension):
            raise N.GlinerDecideError(N.GD_ERR_SHAPE, "queries shape does not match the given dimensions")
        H, L = heads, sequence_length
        c2p, p2c = _indices(c2p_indices, p2c_indices, H, L)
        pk = as_f16(position_key, "position_key").reshape(H, position_count, head_dimension).contiguous()
        pq = as_f16(position_query, "position_query").reshape(H, position_count, head_dimension).contiguous()
        km = as_f16(key_mask, "key_mask").reshape(batch, L).contiguous()
        out = torch.empty((batch, L, H, head_dimension), dtype=torch.float16, device=q.device)
        N.check(self._lib.gd_fused_attention(ptr(q), ptr(k), ptr(v), ptr(pk), ptr(pq), ptr(c2p), ptr(p2c), ptr(km),
                                             float(scale), batch, H, L, head_dimension, position_count, ptr(out),
                                             stream_handle()))
        return out

    # -- default graph: relative bias + masked softmax (+ P.V) --------------
    def deberta_attention(self, q, k, v, position_key, position_query, mask, *, output: str = "context",
                          mask_kind: str = "attention", out: torch.Tensor | None = None,
                          score: str = "default") -> torch.Tensor:
        """Closed-form-index DeBERTa attention (DeBERTa.swift:322-410).

        q, k, v: [B, H, L, D] views with contiguous D (any strides, e.g. the
        split of a fused [B, L, 3, H, D] projection); position_key /
        position_query: [H, P, D] views with contiguous D; mask: [B, L] fp16.
        output: "probs" -> [B, H, L, L]; "context" -> [B, L, H*D];
        "bias" -> the SDPA additive mask [B, H, L, L] (or the kernel bias).
        score: the graph reproduced -- "default" (:374-394), "explicit"
        (useFastAttention = false, :397-409), "kernel_bias"
        (useCustomRelativeKernel, :357-372 + SDPA), "kernel_bias_explicit"
        (both), "fused" (useFusedAttentionKernel, :337-354)."""
        for name, t in (("q", q), ("k", k)) + ((("v", v),) if v is not None else ()):
            if not t.is_cuda or t.dtype != torch.float16 or t.dim() != 4 or t.stride(3) != 1:
                raise N.GlinerDecideError(N.GD_ERR_SHAPE, f"{name} must be a [B, H, L, D] fp16 GPU view with "
                                                          "contiguous D")
        B, H, L, D = q.shape
        for name, t in (("position_key", position_key), ("position_query", position_query)):
            if t.dim() != 3 or t.shape[0] != H or t.shape[2] != D or t.stride(2) != 1 or t.dtype != torch.float16:
                raise N.GlinerDecideError(N.GD_ERR_SHAPE, f"{name} must be a [H, P, D] fp16 view with contiguous D")
        P = position_key.shape[1]
        mask = as_f16(mask, "mask").reshape(B, L).contiguous()
        kind = {"probs": N.GD_ATTN_OUT_PROBS, "context": N.GD_ATTN_OUT_CONTEXT, "bias": N.GD_ATTN_OUT_BIAS}[output]
        sc = {"default": N.GD_ATTN_SCORE_DEFAULT, "explicit": N.GD_ATTN_SCORE_EXPLICIT,
              "kernel_bias": N.GD_ATTN_SCORE_KERNEL_BIAS, "kernel_bias_explicit": N.GD_ATTN_SCORE_KERNEL_BIAS_EXPLICIT,
              "fused": N.GD_ATTN_SCORE_FUSED}[score]
        mk = {"attention": N.GD_MASK_ATTENTION, "additive": N.GD_MASK_ADDITIVE}[mask_kind]
        if out is None:
            shape = (B, L, H * D) if kind == N.GD_ATTN_OUT_CONTEXT else (B, H, L, L)
            out = torch.empty(shape, dtype=torch.float16, device=q.device)
        ldo = H * D if kind == N.GD_ATTN_OUT_CONTEXT else L
        vv = v if v is not None else q
        N.check(self._lib.gd_deberta_attention(
            N.GdBhld(ptr(q), *q.stride()[:3]), N.GdBhld(ptr(k), *k.stride()[:3]),
            N.GdBhld(ptr(vv), *vv.stride()[:3]),
            N.GdTable(ptr(position_key), position_key.stride(0), position_key.stride(1)),
            N.GdTable(ptr(position_query), position_query.stride(0), position_query.stride(1)),
            ptr(mask), mk, B, H, L, D, P, 256, kind | sc, ptr(out), ldo, stream_handle()))
        return out

    # -- default graph: embedding stage (DeBERTa.swift:285-292) -------------
    def embedding_layer_norm(self, ids, attention_mask, table, gamma, beta, eps: float,
                             error_flag: torch.Tensor | None = None) -> torch.Tensor:
        ids = as_i32(ids, "ids")
        B, L = _dims(ids, 2, "ids")
        mask = as_f16(attention_mask, "attention_mask").reshape(B, L).contiguous()
        table = as_f16(table, "table")
        V, Cdim = _dims(table, 2, "table")
        out = torch.empty((B, L, Cdim), dtype=torch.float16, device=ids.device)
        N.check(self._lib.gd_embedding_layer_norm(ptr(ids), ptr(mask), ptr(table), ptr(as_f16(gamma, "gamma")),
                                                  ptr(as_f16(beta, "beta")), ptr(out), B, L, Cdim, V, float(eps),
                                                  ptr(error_flag), stream_handle()))
        return out

    # -- LinearWeight / FusedProjectionWeight (DeBERTa.swift:60-92) ---------
    def linear(self, x, weight, bias=None, epilogue: str = "bias", rows: torch.Tensor | None = None) -> torch.Tensor:
        """epilogue(x W^T + b); epilogue in {"none", "bias", "gelu", "relu"}.
        rows (int32) gathers rows of x first (marker gather)."""
        x = as_f16(x, "x")
        w = as_f16(weight, "weight")
        N_, K = _dims(w, 2, "weight")
        if x.shape[-1] != K:
            raise N.GlinerDecideError(N.GD_ERR_SHAPE, f"x last dim {x.shape[-1]} != weight in-features {K}")
        x2 = x.reshape(-1, K)
        if rows is not None:
            rows = as_i32(rows, "rows").reshape(-1)
            M = rows.numel()
            lead = (M,)
        else:
            M = x2.shape[0]
            lead = tuple(x.shape[:-1])
        epi = {"none": N.GD_EPI_NONE, "bias": N.GD_EPI_BIAS, "gelu": N.GD_EPI_BIAS_GELU,
               "relu": N.GD_EPI_BIAS_RELU}[epilogue]
        b = as_f16(bias, "bias") if bias is not None else None
        out = torch.empty(lead + (N_,), dtype=torch.float16, device=x.device)
        N.check(self._lib.gd_linear(ptr(x2), ptr(w), ptr(b), ptr(out), M, N_, K, K, N_, ptr(rows), x2.shape[0], epi,
                                    stream_handle()))
        return out

    def relative_index_table(self, n: int, device=None) -> torch.Tensor:
        """Device-computed idx(r) for r in [-(n-1), n-1] (DeBERTa.swift:521-551)."""
        out = torch.empty(2 * n - 1, dtype=torch.int32, device=device or torch.device("cuda"))
        N.check(self._lib.gd_relative_index_table(ptr(out), n, 256, 512, stream_handle()))
        return out


def scale_f32(head_size: int) -> float:
    """1 / Float(headSize * 3).squareRoot() (DeBERTa.swift:347)."""
    import numpy as np
    return float(np.float32(1.0) / np.float32(math.sqrt(head_size * 3)))
