"""Numpy restatement of the reference GLiNER-Decide classification graph.

TEST INFRASTRUCTURE ONLY (the checker).  Imported by `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`; never by
the product path.

Reference files (paths relative to the reference repository root):

* `Sources/GLiNERDecideCore/DeBERTa.swift`       -- the model graph
* `Sources/GLiNERDecideCore/FusedKernels.swift`  -- the three Metal kernels
* `Sources/GLiNERDecideCore/Configuration.swift` -- hyper-parameters
* `Sources/gliner-decide-raw/RawCLI.swift`       -- label decode
* `Sources/gliner-decide-metal/main.swift`       -- batch chunking
* `Sources/GLiNERDecideCore/NativeTokenizer.swift` -- bucket rule

Arithmetic model.  The reference runs every op on fp16 MLX arrays; each op
accumulates in fp32 and rounds its output to fp16.  Functions here compute in
float64 (or float32 when `dtype=np.float32` is asked for speed) and, with
`round16=True`, round to fp16 exactly where a reference op writes an fp16
array.  Rounding points *inside* MLX built-ins (SDPA tiling, LayerNorm
internals, erf) are not visible in the reference sources; those are computed
exactly and rounded once at the op output ("parity unpinned at the MLX
boundary" -- the stated tolerances absorb it).

Each function names what pins it ("pinned by"): a closed form, a known-answer
test from the reference, brute force, or an independent library routine
(torch / HF transformers DeBERTa-v2, used only as a cross-check in tests).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

MASK_FILL = -65504.0  # fp16 lowest, DeBERTa.swift:331-335
LOGIT_FILL = -10000.0  # DeBERTa.swift:438-443
DEFAULT_BUCKETS = (32, 64, 96, 128, 256, 512)  # NativeTokenizer.swift:79
POSITION_COUNT = 512  # hard-coded in DeBERTa.swift:505 and :352,:371


# ---------------------------------------------------------------------------
# Configuration -- Configuration.swift:3-48
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Config:
    """`DeBERTaV2Configuration.default` (Configuration.swift:38-48) plus the
    vocabulary size and classifier width, which the reference fixes by the
    checkpoint shape (DeBERTa.swift:199-202) and `classifier.0` (1024->2048).

    pinned by: ConfigurationTests.swift:4-11 (1024/4096/24/16/64).
    """

    hidden_size: int = 1024
    intermediate_size: int = 4096
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    layer_norm_eps: float = 1e-7
    position_buckets: int = 256
    max_relative_positions: int = -1
    hidden_act: str = "gelu"
    pad_token_id: int = 0
    vocab_size: int = 128011
    classifier_hidden: int = 2048

    @property
    def head_size(self) -> int:  # Configuration.swift:36
        return self.hidden_size // self.num_attention_heads


# ---------------------------------------------------------------------------
# Rounding helpers
# ---------------------------------------------------------------------------
def f16(x, enabled: bool = True, dtype=np.float64):
    """Round to IEEE fp16 (round-to-nearest-even, overflow to +-inf) and
    return in the compute dtype."""
    x = np.asarray(x)
    if not enabled:
        return x.astype(dtype, copy=False)
    with np.errstate(over="ignore"):
        return x.astype(np.float16).astype(dtype)


# ---------------------------------------------------------------------------
# Relative positions -- DeBERTa.swift:498-551
# ---------------------------------------------------------------------------
def relative_bucket(relative, bucket_size: int = 256, max_position: int = POSITION_COUNT):
    """Log-bucketed relative position (`makeRelativePositions`,
    DeBERTa.swift:521-551), evaluated in float64 like the Swift `Double` code.

    pinned by: brute-force scalar restatement + the committed table
    `tests/golden/relative_bucket_256_512.npy`; invariants (odd symmetry,
    identity for |r| <= 128, monotone, range +-255); HF transformers
    `make_log_bucket_position` as an independent cross-check.
    """
    r = np.asarray(relative, dtype=np.int64)
    mid = bucket_size // 2
    abs_pos = np.where((r > -mid) & (r < mid), mid - 1, np.abs(r)).astype(np.float64)
    with np.errstate(divide="ignore"):
        log_pos = (
            np.ceil(np.log(abs_pos / mid) / np.log((max_position - 1) / mid) * (mid - 1)).astype(np.int64)
            + mid
        )
    sign = np.where(r < 0, -1, 1)
    return np.where(abs_pos <= mid, r, log_pos * sign).astype(np.int64)


def relative_positions(seq_len: int, bucket_size: int = 256, max_position: int = POSITION_COUNT):
    """`makeRelativePositions` grid: out[q, k] = bucket(q - k), shape [L, L]
    (DeBERTa.swift:529-550)."""
    q = np.arange(seq_len)[:, None]
    k = np.arange(seq_len)[None, :]
    return relative_bucket(q - k, bucket_size, max_position)


def relative_indices(seq_len: int, bucket_size: int = 256):
    """`cachedRelativeData` (DeBERTa.swift:498-519).

    c2p[q, k] = clip(bucket(q - k) + 256, 0, 511)            (:507-510)
    p2c[a, b] = clip(-bucket(a - b) + 256, 0, 511)           (:511-515)

    MLX `transposed(0, 1)` on a 2-D array is the identity permutation, so the
    p2c base is the same [L, L] grid (not its transpose).  Returns two
    [L, L] int64 arrays (the reference broadcasts them to [1, H, L, L]).

    pinned by: HF DeBERTa-v2 `disentangled_attention_bias` index math
    (c2p uses clip(rel + att_span), p2c uses clip(-rel + att_span) on the
    transposed gather) through the layer cross-check in tests; closed form
    p2c[k, q] == c2p[q, k] by odd symmetry of the bucket.
    """
    pos = relative_positions(seq_len, bucket_size)
    span = bucket_size
    c2p = np.clip(pos + span, 0, 2 * span - 1)
    p2c = np.clip(-pos + span, 0, 2 * span - 1)
    return c2p, p2c


# ---------------------------------------------------------------------------
# LayerNorm -- DeBERTa.swift:94-106, FusedKernels.swift:125-155
# ---------------------------------------------------------------------------
def layer_norm(x, gamma, beta, eps: float, round16: bool = True, dtype=np.float64):
    """`LayerNormWeight.callAsFunction` -> `MLXFast.layerNorm` over the last
    axis: (x - mean) / sqrt(var + eps) * gamma + beta, biased variance
    (DeBERTa.swift:103-105).  Output rounded to fp16.

    pinned by: the reference known-answer test main.swift:194-225 (analytic
    mean/variance of x_i = i/1024) and torch.nn.functional.layer_norm.
    """
    x = np.asarray(x, dtype=dtype)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + dtype(eps)) * np.asarray(gamma, dtype) + np.asarray(beta, dtype)
    return f16(y, round16, dtype)


def residual_layer_norm_default(x, residual, gamma, beta, eps: float, round16: bool = True, dtype=np.float64):
    """Default-path residual LayerNorm `norm(x + residual)`
    (DeBERTa.swift:463): the fp16 add rounds the sum before LayerNorm."""
    s = f16(np.asarray(x, dtype) + np.asarray(residual, dtype), round16, dtype)
    return layer_norm(s, gamma, beta, eps, round16, dtype)


def residual_layer_norm_kernel(x, residual, gamma, beta, eps: float, round16: bool = True, dtype=np.float64):
    """`gliner_decide_residual_layer_norm` (FusedKernels.swift:125-155): the
    sum x + residual is formed in fp32 (no fp16 rounding), mean and biased
    variance over C, rsqrt(var + eps), one rounding at the output.

    pinned by: main.swift:194-225 known answer; torch layer_norm of the sum.
    """
    s = np.asarray(x, dtype) + np.asarray(residual, dtype)
    return layer_norm(s, gamma, beta, eps, round16, dtype)


# ---------------------------------------------------------------------------
# Embedding stage -- DeBERTa.swift:285-292
# ---------------------------------------------------------------------------
def embedding(ids, attention_mask, table, gamma, beta, eps: float, round16: bool = True, dtype=np.float64):
    """x = E[ids]; x = LN(x); x = x * mask (mask cast to fp16)
    (DeBERTa.swift:285-292).  No position or token-type embeddings."""
    ids = np.asarray(ids, dtype=np.int64)
    x = np.asarray(table)[ids].astype(dtype)
    x = layer_norm(x, gamma, beta, eps, round16, dtype)
    m = f16(np.asarray(attention_mask, dtype), round16, dtype)
    return f16(x * m[..., None], round16, dtype)


# ---------------------------------------------------------------------------
# Dense layers
# ---------------------------------------------------------------------------
def linear(x, weight, bias, round16: bool = True, dtype=np.float64):
    """`LinearWeight` / `FusedProjectionWeight`: addMM(b, x, W^T), W stored
    [out, in] (DeBERTa.swift:60-92).  One rounding of (x W^T + b).

    pinned by: numpy matmul (library) -- the formula is the definition.
    """
    x = np.asarray(x, dtype)
    w = np.asarray(weight, dtype)
    y = x @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype)
    return f16(y, round16, dtype)


def gelu(x, round16: bool = True, dtype=np.float64):
    """MLXNN.gelu, exact erf form x * (1 + erf(x / sqrt 2)) / 2
    (DeBERTa.swift:421).  Computed exactly and rounded once (MLX's internal
    rounding of the elementwise chain is not visible in the reference).

    pinned by: torch.nn.functional.gelu(approximate='none').
    """
    x = np.asarray(x, dtype)
    erf = np.vectorize(math.erf, otypes=[np.float64]) if x.size < 4096 else _erf_np
    y = 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))
    return f16(y, round16, dtype)


def _erf_np(x):
    """Vectorised erf via scipy when present (tests), else math.erf."""
    try:
        from scipy.special import erf as _erf
    except ImportError:  # pragma: no cover
        return np.vectorize(math.erf, otypes=[np.float64])(x)
    return _erf(x)


# ---------------------------------------------------------------------------
# Relative bias -- DeBERTa.swift:374-379 and FusedKernels.swift:83-123
# ---------------------------------------------------------------------------
def scale_f16(head_size: int) -> float:
    """MLXArray(Float(headSize * 3).squareRoot(), dtype: .float16)
    (DeBERTa.swift:323-326): 13.859375 for head size 64."""
    return float(np.float16(math.sqrt(head_size * 3)))


def scale_f32(head_size: int) -> float:
    """1 / Float(headSize * 3).squareRoot() as fp32 (DeBERTa.swift:347,390)."""
    return float(np.float32(1.0) / np.float32(math.sqrt(head_size * 3)))


def relative_bias_default(q, k, pos_key, pos_query, c2p_idx, p2c_idx, head_size: int, round16: bool = True,
                          dtype=np.float64, bias_scale: float | None = None):
    """Default MLX relative bias (DeBERTa.swift:374-379).

    q, k: [B, H, L, D]; pos_key/pos_query: [H, P, D]; c2p_idx, p2c_idx: [L, L].
    c2pRaw = q @ posK^T  -> fp16               (:374)
    c2p[q,k] = c2pRaw[q, c2p_idx[q,k]]         (:375, takeAlong axis -1)
    p2cRaw = k @ posQ^T  -> fp16               (:376)
    p2c[q,k] = p2cRaw[k, p2c_idx[k,q]]         (:377-378, takeAlong then swap last two axes)
    bias = fp16(fp16(c2p + p2c) / fp16(sqrt(3 D)))   (:379)
    Returns bias [B, H, L, L].  `bias_scale` overrides the fp16 scale (only
    for cross-checks against implementations that divide by the fp32 value).

    pinned by: brute-force per-element loops (tests), the reference
    procedural known-answer test main.swift:141-192, and the HF DeBERTa-v2
    layer cross-check.
    """
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    pk = np.asarray(pos_key, dtype)
    pq = np.asarray(pos_query, dtype)
    c2p_raw = f16(np.matmul(q, np.swapaxes(pk, -1, -2)[None]), round16, dtype)
    p2c_raw = f16(np.matmul(k, np.swapaxes(pq, -1, -2)[None]), round16, dtype)
    L = q.shape[2]
    rows = np.arange(L)[:, None]
    c2p = c2p_raw[:, :, rows, np.asarray(c2p_idx)]  # [B,H,L,L]: [q, c2p_idx[q,k]]
    g = p2c_raw[:, :, rows, np.asarray(p2c_idx)]  # [B,H,L,L]: [a, p2c_idx[a,b]]
    p2c = np.swapaxes(g, -1, -2)
    s = f16(c2p + p2c, round16, dtype)
    scale = scale_f16(head_size) if bias_scale is None else bias_scale
    return f16(s / scale, round16, dtype)


def relative_bias_kernel(q, k, pos_key, pos_query, c2p_indices, p2c_indices, key_mask, scale: float,
                         round16: bool = True):
    """`gliner_decide_relative_bias` (FusedKernels.swift:83-123) with general
    index tensors.

    q, k: [B, H, L, D]; pos_key/pos_query: [1 or H, P, D] flattened as
    (h*P + idx)*D + d; c2p_indices/p2c_indices: [H, L, L] read as
    c2p[(h*L + q)*L + k] and p2c[(h*L + k)*L + q]; key_mask [B, L] additive
    (masked iff < -60000).  score = (c2p + p2c) * scale in fp32, masked keys
    := -65504, output fp16 [B, H, L, L].

    pinned by: the reference known-answer test main.swift:141-192 restated
    with its exact generators, and brute-force loops.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    B, H, L, D = q.shape
    pk = np.asarray(pos_key, np.float64).reshape(H, -1, D)
    pq = np.asarray(pos_query, np.float64).reshape(H, -1, D)
    c2pi = np.broadcast_to(np.asarray(c2p_indices), (H, L, L))
    p2ci = np.broadcast_to(np.asarray(p2c_indices), (H, L, L))
    hh = np.arange(H)[:, None, None]
    gk = pk[hh, c2pi]  # [H, L(q), L(k), D]
    gq = pq[hh, np.swapaxes(p2ci, 1, 2)]  # [H, L(q), L(k), D] at p2c[h, k, q]
    c2p = np.einsum("bhqd,hqkd->bhqk", q, gk, optimize=True)
    p2c = np.einsum("bhkd,hqkd->bhqk", k, gq, optimize=True)
    score = (c2p + p2c) * np.float64(np.float32(scale))
    masked = np.asarray(key_mask, np.float64).reshape(B, 1, 1, L) < -60000.0
    score = np.where(masked, MASK_FILL, score)
    return f16(score, round16)


# ---------------------------------------------------------------------------
# Attention -- DeBERTa.swift:382-409, FusedKernels.swift:13-81
# ---------------------------------------------------------------------------
def _softmax(x, axis=-1):
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def additive_key_mask(attention_mask):
    """valid = mask > 0 -> additive 0 / -65504 fp16, shape [B, 1, 1, L]
    (DeBERTa.swift:329-335)."""
    valid = np.asarray(attention_mask, np.float64) > 0
    return np.where(valid, 0.0, MASK_FILL)[:, None, None, :]


def attention_probs_default(q, k, bias, attention_mask, head_size: int, round16: bool = True, dtype=np.float64):
    """Probabilities of the default fast-attention path (DeBERTa.swift:382-392):
    mask = fp16(bias + additiveKeyMask) (fp16 add, may overflow to -inf);
    P = softmax(q k^T * (1/sqrt(3D)) + mask) in fp32-or-better.
    Returns P [B, H, L, L] (unrounded)."""
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    mask = f16(np.asarray(bias, dtype) + additive_key_mask(attention_mask), round16, dtype)
    scores = np.matmul(q, np.swapaxes(k, -1, -2)) * dtype(scale_f32(head_size)) + mask
    with np.errstate(over="ignore", invalid="ignore"):
        return _softmax(scores)


def attention_default(q, k, v, bias, attention_mask, head_size: int, round16: bool = True, dtype=np.float64):
    """MLXFast.scaledDotProductAttention with the additive bias+key mask,
    then transpose/reshape to [B, L, H*D] (DeBERTa.swift:382-395).  Key-only
    masking: padded query rows attend over the valid keys."""
    p = attention_probs_default(q, k, bias, attention_mask, head_size, round16, dtype)
    ctx = np.matmul(p, np.asarray(v, dtype))
    B, H, L, D = ctx.shape
    return f16(np.transpose(ctx, (0, 2, 1, 3)).reshape(B, L, H * D), round16, dtype)


def attention_sdpa_mask(q, k, v, mask, head_size: int, round16: bool = True, dtype=np.float64):
    """MLXFast.scaledDotProductAttention with `mask` as the whole additive
    mask (DeBERTa.swift:382-395): softmax(q k^T * (1/sqrt(3D)) + mask) v,
    transposed to [B, L, H*D].  The useCustomRelativeKernel graph passes the
    kernel's bias (masked keys already -65504) with no key mask added
    (:383-385)."""
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    scores = np.matmul(q, np.swapaxes(k, -1, -2)) * dtype(scale_f32(head_size)) + np.asarray(mask, dtype)
    with np.errstate(over="ignore", invalid="ignore"):
        p = _softmax(scores)
    ctx = np.matmul(p, np.asarray(v, dtype))
    B, H, L, D = ctx.shape
    return f16(np.transpose(ctx, (0, 2, 1, 3)).reshape(B, L, H * D), round16, dtype)


def attention_generic(q, k, v, bias, attention_mask, head_size: int, round16: bool = True, dtype=np.float64,
                      where_mask: bool = True, content_scale: float | None = None):
    """Explicit-score path (`useFastAttention = false`, `--generic-attention`,
    DeBERTa.swift:397-409):
    content = fp16(fp16(q k^T) / fp16(sqrt(3 D)))   (:399, MLX fp16 matmul then fp16 divide)
    scores  = fp16(content + bias)                   (:400)
    masked keys := -65504 (`where`, :401-407; skipped with where_mask=False,
    the useCustomRelativeKernel graph, whose bias already holds -65504)
    P = fp16(softmax(scores)) (:407); ctx = fp16(P v) (:408) -> [B, L, H*D].
    `content_scale` overrides fp16(sqrt(3 D)) (exact cross-checks only).

    pinned by: scalar loops with explicit fp16 rounding at every op (tests),
    and, with round16=False, the HF DeBERTa-v2 layer (float64).
    """
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    cs = scale_f16(head_size) if content_scale is None else content_scale
    content = f16(f16(np.matmul(q, np.swapaxes(k, -1, -2)), round16, dtype) / cs, round16, dtype)
    with np.errstate(over="ignore"):
        scores = f16(content + np.asarray(bias, dtype), round16, dtype)
    if where_mask:
        valid = (np.asarray(attention_mask, np.float64) > 0)[:, None, None, :]
        scores = np.where(valid, scores, MASK_FILL)
    with np.errstate(over="ignore", invalid="ignore"):
        p = f16(_softmax(scores), round16, dtype)
    ctx = f16(np.matmul(p, np.asarray(v, dtype)), round16, dtype)
    B, H, L, D = ctx.shape
    return np.transpose(ctx, (0, 2, 1, 3)).reshape(B, L, H * D)


def fused_attention_kernel(q, k, v, pos_key, pos_query, c2p_indices, p2c_indices, key_mask, scale: float,
                           round16: bool = True):
    """`gliner_decide_fused_attention` (FusedKernels.swift:13-81):
    score = (q.k + q.posK[c2p] + k.posQ[p2c]) * scale (fp32), masked keys
    (key_mask < -60000) := -65504, softmax with the running max seeded at
    -65504, out[b, q, h, :] = sum_k w_k v_k -> [B, L, H, D] fp16.

    pinned by: brute-force loops on tiny shapes (tests) and torch SDPA with
    an explicit additive bias.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, L, D = q.shape
    # The kernel keeps qk + c2p + p2c in fp32: no intermediate fp16 rounding.
    pk = np.asarray(pos_key, np.float64).reshape(H, -1, D)
    pq = np.asarray(pos_query, np.float64).reshape(H, -1, D)
    c2pi = np.broadcast_to(np.asarray(c2p_indices), (H, L, L))
    p2ci = np.broadcast_to(np.asarray(p2c_indices), (H, L, L))
    hh = np.arange(H)[:, None, None]
    c2p = np.einsum("bhqd,hqkd->bhqk", q, pk[hh, c2pi], optimize=True)
    p2c = np.einsum("bhkd,hqkd->bhqk", k, pq[hh, np.swapaxes(p2ci, 1, 2)], optimize=True)
    score = (np.matmul(q, np.swapaxes(k, -1, -2)) + c2p + p2c) * np.float64(np.float32(scale))
    masked = np.asarray(key_mask, np.float64).reshape(B, 1, 1, L) < -60000.0
    score = np.where(masked, MASK_FILL, score)
    m = np.maximum(score.max(axis=-1, keepdims=True), MASK_FILL)
    e = np.exp(score - m)
    w = e / e.sum(axis=-1, keepdims=True)
    out = np.matmul(w, v).transpose(0, 2, 1, 3)
    return f16(out, round16)


def attention_stage(q, k, v, pos_key, pos_query, attention_mask, head_size: int, *, fast: bool = True,
                    custom_bias: bool = False, fused: bool = False, round16: bool = True, dtype=np.float64,
                    bias_scale: float | None = None):
    """The attention stage of `forward` under the classifier's flags
    (DeBERTa.swift:322-410); q, k, v [B, H, L, D], tables [H, P, D] ->
    context [B, L, H*D].

    fused (useFusedAttentionKernel, :337-354): the fused Metal kernel, score
        (q.k + c2p + p2c) * (1/sqrt(3D)) in fp32, its output [B, L, H, D]
        reshaped.
    custom_bias (useCustomRelativeKernel, :357-372): the relative-bias Metal
        kernel (fp32 c2p + p2c times the fp32 scale, masked keys -65504, fp16)
        replaces the default bias; with `fast` it is the whole SDPA mask
        (:383-385), else it is added to the content score with no `where`
        (:401-403).
    otherwise the default bias (:374-379), then SDPA with bias + key mask
    (`fast`, :383-394) or the explicit-score path (:397-409).
    `bias_scale` replaces both fp16(sqrt(3D)) divisors (exact cross-checks
    against HF, which divides by the fp32 value).

    pinned by: its pieces' pins (Metal-kernel known answers, brute force,
    torch SDPA) and, with round16=False, the HF DeBERTa-v2 layer for every
    flag combination (the flags change rounding points and masking, not the
    exact mathematics).
    """
    B, H, L, D = np.shape(q)
    c2p_idx, p2c_idx = relative_indices(L)
    key_mask = additive_key_mask(attention_mask)[:, 0, 0, :]
    if fused:
        out = fused_attention_kernel(q, k, v, pos_key, pos_query, c2p_idx, p2c_idx, key_mask, scale_f32(D),
                                     round16=round16)
        return np.asarray(out, dtype).reshape(B, L, H * D)
    if custom_bias:
        scale = scale_f32(D) if bias_scale is None else 1.0 / bias_scale
        bias = np.asarray(relative_bias_kernel(q, k, pos_key, pos_query, c2p_idx, p2c_idx, key_mask, scale,
                                               round16=round16), dtype)
        if fast:
            return attention_sdpa_mask(q, k, v, bias, D, round16, dtype)
        return attention_generic(q, k, v, bias, attention_mask, D, round16, dtype, where_mask=False,
                                 content_scale=bias_scale)
    bias = relative_bias_default(q, k, pos_key, pos_query, c2p_idx, p2c_idx, D, round16, dtype, bias_scale)
    if fast:
        return attention_default(q, k, v, bias, attention_mask, D, round16, dtype)
    return attention_generic(q, k, v, bias, attention_mask, D, round16, dtype, content_scale=bias_scale)


# ---------------------------------------------------------------------------
# Weights -- DeBERTa.swift:118-150, 197-241
# ---------------------------------------------------------------------------
@dataclass
class LayerWeights:
    qkv_w: np.ndarray  # [3C, C]   query_proj;key_proj;value_proj (DeBERTa.swift:129-136)
    qkv_b: np.ndarray  # [3C]
    out_w: np.ndarray  # [C, C]    attention.output.dense
    out_b: np.ndarray
    ln1_g: np.ndarray  # attention.output.LayerNorm
    ln1_b: np.ndarray
    inter_w: np.ndarray  # [F, C]  intermediate.dense
    inter_b: np.ndarray
    ffn_out_w: np.ndarray  # [C, F] output.dense
    ffn_out_b: np.ndarray
    ln2_g: np.ndarray  # output.LayerNorm
    ln2_b: np.ndarray


@dataclass
class ModelWeights:
    word_embeddings: np.ndarray  # [V, C]
    emb_ln_g: np.ndarray
    emb_ln_b: np.ndarray
    rel_embeddings: np.ndarray  # [512, C]
    rel_ln_g: np.ndarray
    rel_ln_b: np.ndarray
    layers: list = field(default_factory=list)
    cls0_w: np.ndarray = None  # [2048, C]
    cls0_b: np.ndarray = None
    cls2_w: np.ndarray = None  # [1, 2048]
    cls2_b: np.ndarray = None

    @classmethod
    def from_store(cls, store: dict, config: Config) -> "ModelWeights":
        """Assemble from a key -> array mapping with the checkpoint key names
        (DeBERTa.swift:127-149, 199-208, 228-229)."""
        def get(key):
            if key not in store:
                raise KeyError(f"Missing model weight: {key}")
            return np.asarray(store[key])

        layers = []
        for i in range(config.num_hidden_layers):
            p = f"encoder.encoder.layer.{i}"
            qkv_w = np.concatenate([get(f"{p}.attention.self.{n}_proj.weight") for n in ("query", "key", "value")], 0)
            qkv_b = np.concatenate([get(f"{p}.attention.self.{n}_proj.bias") for n in ("query", "key", "value")], 0)
            layers.append(LayerWeights(
                qkv_w=qkv_w, qkv_b=qkv_b,
                out_w=get(f"{p}.attention.output.dense.weight"), out_b=get(f"{p}.attention.output.dense.bias"),
                ln1_g=get(f"{p}.attention.output.LayerNorm.weight"), ln1_b=get(f"{p}.attention.output.LayerNorm.bias"),
                inter_w=get(f"{p}.intermediate.dense.weight"), inter_b=get(f"{p}.intermediate.dense.bias"),
                ffn_out_w=get(f"{p}.output.dense.weight"), ffn_out_b=get(f"{p}.output.dense.bias"),
                ln2_g=get(f"{p}.output.LayerNorm.weight"), ln2_b=get(f"{p}.output.LayerNorm.bias"),
            ))
        return cls(
            word_embeddings=get("encoder.embeddings.word_embeddings.weight"),
            emb_ln_g=get("encoder.embeddings.LayerNorm.weight"), emb_ln_b=get("encoder.embeddings.LayerNorm.bias"),
            rel_embeddings=get("encoder.encoder.rel_embeddings.weight"),
            rel_ln_g=get("encoder.encoder.LayerNorm.weight"), rel_ln_b=get("encoder.encoder.LayerNorm.bias"),
            layers=layers,
            cls0_w=get("classifier.0.weight"), cls0_b=get("classifier.0.bias"),
            cls2_w=get("classifier.2.weight"), cls2_b=get("classifier.2.bias"),
        )


def relative_tables(weights: ModelWeights, config: Config, round16: bool = True, dtype=np.float64):
    """Init-time relative precompute (DeBERTa.swift:204-227): relN = LN(rel)
    [512, C]; per layer [posQ | posK] = relN [Wq; Wk]^T + [bq; bk] -> [512, 2C],
    reshaped [1, 512, 2, H, D] and split, each transposed to [H, 512, D].
    Returns a list of (pos_query, pos_key) per layer."""
    C, H, D = config.hidden_size, config.num_attention_heads, config.head_size
    rel_n = layer_norm(weights.rel_embeddings, weights.rel_ln_g, weights.rel_ln_b, config.layer_norm_eps,
                       round16, dtype)
    out = []
    for lw in weights.layers:
        qk = linear(rel_n, lw.qkv_w[: 2 * C], lw.qkv_b[: 2 * C], round16, dtype)  # [512, 2C]
        qk = qk.reshape(POSITION_COUNT, 2, H, D)
        out.append((np.transpose(qk[:, 0], (1, 0, 2)), np.transpose(qk[:, 1], (1, 0, 2))))
    return out


# ---------------------------------------------------------------------------
# Forward -- DeBERTa.swift:274-447
# ---------------------------------------------------------------------------
def encoder_layer(hidden, lw: LayerWeights, pos_query, pos_key, attention_mask, config: Config,
                  round16: bool = True, dtype=np.float64, use_fused_kernels: bool = False,
                  return_intermediates: bool = False, bias_scale: float | None = None,
                  use_fast_attention: bool = True, use_custom_relative_kernel: bool = False,
                  use_fused_attention_kernel: bool = False):
    """One DeBERTa layer of `forward` (DeBERTa.swift:296-428).
    hidden [B, L, C] -> [B, L, C].

    The flags mirror GLiNERDecideClassifier.init (DeBERTa.swift:188-196):
    the attention stage follows `attention_stage`; the residual LayerNorms use
    the Metal kernel (fp32 sum, FusedKernels residual LN) whenever the
    reference holds a FusedKernels instance, i.e. when any of
    use_fused_kernels, use_custom_relative_kernel or use_fused_attention_kernel
    is set (:230-232, :449-462); otherwise the fp16 sum `norm(x + residual)`.
    """
    use_fused_kernels = use_fused_kernels or use_custom_relative_kernel or use_fused_attention_kernel
    B, L, C = hidden.shape
    H, D = config.num_attention_heads, config.head_size
    eps = config.layer_norm_eps
    hidden = np.asarray(hidden, dtype)
    qkv = linear(hidden, lw.qkv_w, lw.qkv_b, round16, dtype).reshape(B, L, 3, H, D)
    q = np.transpose(qkv[:, :, 0], (0, 2, 1, 3))
    k = np.transpose(qkv[:, :, 1], (0, 2, 1, 3))
    v = np.transpose(qkv[:, :, 2], (0, 2, 1, 3))
    ctx = attention_stage(q, k, v, pos_key, pos_query, attention_mask, D, fast=use_fast_attention,
                          custom_bias=use_custom_relative_kernel, fused=use_fused_attention_kernel, round16=round16,
                          dtype=dtype, bias_scale=bias_scale)
    res_ln = residual_layer_norm_kernel if use_fused_kernels else residual_layer_norm_default
    attn_out = linear(ctx, lw.out_w, lw.out_b, round16, dtype)
    h1 = res_ln(attn_out, hidden, lw.ln1_g, lw.ln1_b, eps, round16, dtype)
    inter = gelu(linear(h1, lw.inter_w, lw.inter_b, round16, dtype), round16, dtype)
    ffn = linear(inter, lw.ffn_out_w, lw.ffn_out_b, round16, dtype)
    h2 = res_ln(ffn, h1, lw.ln2_g, lw.ln2_b, eps, round16, dtype)
    if return_intermediates:
        return h2, dict(qkv=qkv.reshape(B, L, 3 * C), ctx=ctx, attn_out=attn_out, h1=h1, inter=inter, ffn=ffn)
    return h2


def classifier_head(hidden, marker_indices, marker_mask, weights: ModelWeights, round16: bool = True,
                    dtype=np.float64):
    """Classifier stage (DeBERTa.swift:430-444): gather marker rows at
    marker_indices + b*L, Linear(C->2048) -> ReLU -> Linear(2048->1), then
    where(marker_mask > 0, v, -10000).  Returns logits [B, Hh, O]."""
    B, L, C = hidden.shape
    mi = np.asarray(marker_indices, np.int64)
    flat = (mi + (np.arange(B) * L)[:, None, None]).reshape(-1)
    m = np.asarray(hidden, dtype).reshape(B * L, C)[flat]
    h = np.maximum(linear(m, weights.cls0_w, weights.cls0_b, round16, dtype), 0.0)
    v = linear(h, weights.cls2_w, weights.cls2_b, round16, dtype)[:, 0].reshape(mi.shape)
    mm = np.asarray(marker_mask, np.float64)
    return f16(np.where(mm > 0, v, LOGIT_FILL), round16, dtype)


class OracleModel:
    """CPU restatement of `GLiNERDecideClassifier` (DeBERTa.swift:156-447).

    `forward` returns logits [B, Hh, O]; `encode` returns the final hidden
    states [B, L, C].  Rows are independent, so callers may evaluate a
    subset of rows of a large batch.
    """

    def __init__(self, weights: ModelWeights, config: Config, round16: bool = True, dtype=np.float64,
                 use_fused_kernels: bool = False, bias_scale: float | None = None, use_fast_attention: bool = True,
                 use_custom_relative_kernel: bool = False, use_fused_attention_kernel: bool = False):
        self.w = weights
        self.config = config
        self.round16 = round16
        self.dtype = dtype
        self.use_fused_kernels = use_fused_kernels
        self.bias_scale = bias_scale
        self.flags = dict(use_fast_attention=use_fast_attention, use_custom_relative_kernel=use_custom_relative_kernel,
                          use_fused_attention_kernel=use_fused_attention_kernel)
        self.tables = relative_tables(weights, config, round16, dtype)

    def embed(self, ids, attention_mask):
        c = self.config
        return embedding(ids, attention_mask, self.w.word_embeddings, self.w.emb_ln_g, self.w.emb_ln_b,
                         c.layer_norm_eps, self.round16, self.dtype)

    def encode(self, ids, attention_mask, num_layers: int | None = None):
        h = self.embed(ids, attention_mask)
        n = self.config.num_hidden_layers if num_layers is None else num_layers
        for i in range(n):
            pq, pk = self.tables[i]
            h = encoder_layer(h, self.w.layers[i], pq, pk, attention_mask, self.config, self.round16,
                              self.dtype, self.use_fused_kernels, bias_scale=self.bias_scale, **self.flags)
        return h

    def forward(self, ids, attention_mask, marker_indices, marker_mask):
        h = self.encode(ids, attention_mask)
        return classifier_head(h, marker_indices, marker_mask, self.w, self.round16, self.dtype)


# ---------------------------------------------------------------------------
# Host-side rules: decode, chunking, buckets
# ---------------------------------------------------------------------------
def decode(logits_row, tasks):
    """`decode` (RawCLI.swift:182-223) for one row.

    logits_row: [Hh, O] (fp32); tasks: list of (num_labels, multi_label).
    Single-label: max-shifted softmax over the task's labels, argmax (first
    maximum, as Swift `max(by:)`).  Multi-label: sigmoid, select p >= 0.5,
    argmax fallback when empty.  Returns [(selected_indices, probabilities)].

    pinned by: closed form; hand-computed cases in tests.
    """
    out = []
    for head, (n, multi) in enumerate(tasks):
        x = np.asarray(logits_row[head, :n], np.float64)
        if multi:
            p = 1.0 / (1.0 + np.exp(-x))
            sel = [i for i in range(n) if p[i] >= 0.5]
            if not sel:
                sel = [int(np.argmax(p))]
        else:
            e = np.exp(x - x.max())
            p = e / e.sum()
            sel = [int(np.argmax(p))]
        out.append((sel, p))
    return out


def select_bucket(length: int, buckets=DEFAULT_BUCKETS) -> int:
    """Smallest bucket >= length among the sorted unique buckets
    (NativeTokenizer.swift:85-88, 134-138); ValueError when none fits."""
    ordered = sorted(set(buckets))
    for b in ordered:
        if b >= length:
            return b
    raise ValueError(f"input of length {length} does not fit buckets {ordered}")


def make_batch_chunk(arrays: dict, start: int, end: int, pad_to: int):
    """`makeBatchChunk` (main.swift:7-51): rows [start, end); when fewer than
    pad_to rows, pad with copies of the last valid row.  Returns
    (chunk dict, valid_count)."""
    valid = end - start
    chunk = {k: np.asarray(v)[start:end] for k, v in arrays.items()}
    if valid >= pad_to:
        return chunk, valid
    pad = pad_to - valid
    out = {}
    for k, v in chunk.items():
        last = v[valid - 1: valid]
        out[k] = np.concatenate([v, np.repeat(last, pad, axis=0)], axis=0)
    return out, valid
