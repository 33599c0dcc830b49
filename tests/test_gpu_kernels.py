"""GPU parity of the standalone kernels against the oracle (through the C-ABI).

Tolerances (fp16 outputs, fp32 arithmetic on the GPU vs float64 in the
oracle with the same fp16 rounding points): an element may differ by at most
one fp16 ulp of the expected value, because fp32 vs float64 accumulation can
move a value across a rounding boundary; integer/index outputs are exact.
Attention probabilities: |dP| <= 1e-3 absolute.
"""

import numpy as np
import pytest
import torch

from oracle import deberta as O

pytestmark = pytest.mark.gpu


def fk():
    from gliner_decide.fused_kernels import FusedKernels
    return FusedKernels()


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def host(t):
    torch.cuda.synchronize()
    return t.detach().float().cpu().numpy().astype(np.float64)


def ulp16(x):
    x = np.abs(np.asarray(x, np.float64))
    x = np.maximum(x, 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(x)) - 10)


def assert_within_ulp(got, want, n_ulp=1.0, max_frac_off=None):
    diff = np.abs(got - want)
    bound = n_ulp * ulp16(want) + 1e-12
    bad = diff > bound
    assert not bad.any(), f"{bad.sum()} elements off by > {n_ulp} ulp; worst {diff.max():.3g}"
    if max_frac_off is not None:
        frac = np.mean(diff > 0)
        assert frac <= max_frac_off, f"{frac:.2e} of elements differ"


# ---------------------------------------------------------------------------
# relative index table (DeBERTa.swift:498-551) -- exact
# ---------------------------------------------------------------------------
def test_relative_index_table_exact(golden):
    table = golden("relative_bucket_256_512.npy")
    got = fk().relative_index_table(512).cpu().numpy()
    np.testing.assert_array_equal(got, np.clip(table + 256, 0, 511))
    got32 = fk().relative_index_table(32).cpu().numpy()
    np.testing.assert_array_equal(got32, np.clip(O.relative_bucket(np.arange(-31, 32)) + 256, 0, 511))


# ---------------------------------------------------------------------------
# residual LayerNorm (FusedKernels.swift:125-155, DeBERTa.swift:463)
# ---------------------------------------------------------------------------
def test_layer_norm_known_answer(golden):
    g = golden("ln_known_answer.npz")
    x = dev(g["x"].reshape(1, 1024))
    ones = torch.ones(1024, dtype=torch.float16, device="cuda")
    zeros = torch.zeros(1024, dtype=torch.float16, device="cuda")
    out = host(fk().residual_layer_norm(x, torch.zeros_like(x), ones, zeros, 1e-7))
    np.testing.assert_array_equal(out[0], g["expected"].astype(np.float16).astype(np.float64))


@pytest.mark.parametrize("round_sum", [False, True])
def test_residual_ln_full_size(round_sum):
    from gliner_decide.synthetic import residual_ln_inputs
    d = residual_ln_inputs(seed=2)
    args = [dev(d[k]) for k in ("x", "residual", "gamma", "beta")]
    out = host(fk().residual_layer_norm(*args, 1e-7, round_sum_f16=round_sum))
    ref_fn = O.residual_layer_norm_default if round_sum else O.residual_layer_norm_kernel
    want = ref_fn(d["x"], d["residual"], d["gamma"], d["beta"], 1e-7)
    assert_within_ulp(out, want, 1.0, max_frac_off=1e-3)


@pytest.mark.parametrize("rows,cols", [(0, 1024), (1, 1024), (7, 512), (5, 2048), (3, 72), (9, 8), (33, 1000)])
def test_residual_ln_shapes(rows, cols):
    r = np.random.default_rng(rows * 7 + cols)
    x = r.standard_normal((rows, cols)).astype(np.float16)
    res = r.standard_normal((rows, cols)).astype(np.float16)
    g = (1 + 0.1 * r.standard_normal(cols)).astype(np.float16)
    b = (0.1 * r.standard_normal(cols)).astype(np.float16)
    out = host(fk().residual_layer_norm(dev(x), dev(res), dev(g), dev(b), 1e-7))
    assert_within_ulp(out, O.residual_layer_norm_kernel(x, res, g, b, 1e-7), 1.0)
    plain = host(fk().residual_layer_norm(dev(x), None, dev(g), dev(b), 1e-7))
    assert_within_ulp(plain, O.layer_norm(x, g, b, 1e-7), 1.0)


def test_residual_ln_in_place():
    """out aliasing residual (how the encoder updates its hidden state)."""
    from gliner_decide import _native as N
    from gliner_decide.device import stream_handle
    r = np.random.default_rng(1)
    x = r.standard_normal((64, 1024)).astype(np.float16)
    res = r.standard_normal((64, 1024)).astype(np.float16)
    g = np.ones(1024, np.float16)
    b = np.zeros(1024, np.float16)
    tx, tr, tg, tb = dev(x), dev(res), dev(g), dev(b)
    N.check(N.lib().gd_residual_layer_norm(tx.data_ptr(), tr.data_ptr(), tg.data_ptr(), tb.data_ptr(), tr.data_ptr(),
                                           64, 1024, 1e-7, N.GD_LN_SUM_F16, stream_handle()))
    assert_within_ulp(host(tr), O.residual_layer_norm_default(x, res, g, b, 1e-7), 1.0)


# ---------------------------------------------------------------------------
# embedding (DeBERTa.swift:285-292)
# ---------------------------------------------------------------------------
def test_embedding_layer_norm():
    r = np.random.default_rng(4)
    V, C, B, L = 3000, 1024, 3, 48
    table = (0.02 * r.standard_normal((V, C))).astype(np.float16)
    g = (1 + 0.02 * r.standard_normal(C)).astype(np.float16)
    b = (0.02 * r.standard_normal(C)).astype(np.float16)
    ids = r.integers(0, V, size=(B, L)).astype(np.int32)
    mask = np.ones((B, L), np.float16)
    mask[1, 30:] = 0
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = host(fk().embedding_layer_norm(dev(ids), dev(mask), dev(table), dev(g), dev(b), 1e-7, flag))
    assert_within_ulp(out, O.embedding(ids, mask, table, g, b, 1e-7), 1.0)
    assert int(flag.item()) == 0
    ids[0, 0] = V + 5  # out of range: reads row 0 and raises the flag
    out = host(fk().embedding_layer_norm(dev(ids), dev(mask), dev(table), dev(g), dev(b), 1e-7, flag))
    assert int(flag.item()) == 1
    ids[0, 0] = 0
    assert_within_ulp(out, O.embedding(ids, mask, table, g, b, 1e-7), 1.0)


# ---------------------------------------------------------------------------
# linear (DeBERTa.swift:60-92, 421, 437)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(1, 128, 64), (65, 256, 128), (300, 1024, 1024), (1000, 384, 192),
                                   (160, 1024, 4096), (160, 4096, 1024), (37, 2048, 1024),
                                   (4096, 1024, 256), (4896, 1024, 4096),  # one round of 160x128 tiles
                                   (5000, 1024, 64), (4920, 1024, 128), (4850, 1024, 192),  # ... 1-3 K steps
                                   (4896, 3072, 1024), (4200, 3072, 64), (5100, 3072, 128),  # QKV: one round of 256x256
                                   (8192, 3072, 1024), (8192, 4096, 1024),
                                   (4896, 4096, 256), (5500, 3072, 256),  # split: whole rounds + 128x128 rest
                                   (4100, 4096, 128), (5120, 4096, 128),  # GELU: one round of 320x256 tiles
                                   (4896, 4096, 64), (4200, 4096, 192),  # ... one and three K steps
                                   (4096, 4096, 64), (4096, 4096, 128), (8192, 4096, 192),  # 256 x 256: 1-3 K steps
                                   (8192, 3072, 64),  # 256 x 192, one K step
                                   (792, 3072, 1024), (1100, 4096, 1024), (1400, 3072, 1024),  # up to 4,096
                                   (1800, 4096, 1024), (2300, 2048, 1024), (2600, 1024, 1024),  # rows: the
                                   (3500, 3072, 1024),  # cost-model tile choice
                                   (9500, 4096, 1024), (11835, 1024, 4096),  # 320 x 256 (GELU) and
                                   (16384, 3072, 1024),  # 256 x 256 tiles over several rounds
                                   (32, 3072, 1024), (7, 4096, 1024),  # one short sequence (32 x 16 tiles)
                                   (17, 1024, 4096), (32, 128, 128), (5, 256, 384)])  # ... one and three K stages
@pytest.mark.parametrize("epi", ["bias", "gelu", "relu", "none"])
def test_linear(m, n, k, epi):
    r = np.random.default_rng(m + n + k)
    x = r.standard_normal((m, k)).astype(np.float16)
    w = (r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16)
    b = r.standard_normal(n).astype(np.float16)
    out = host(fk().linear(dev(x), dev(w), dev(b) if epi != "none" else None, epilogue=epi))
    check_linear(out, x, w, b, epi)


def check_linear(out, x, w, b, epi):
    """|gpu - exact| <= fp16 output rounding + fp32 accumulation error.

    The accumulation term is the standard dot-product bound with a
    sqrt(K) growth factor: 4 sqrt(K) 2^-24 sum_k |x_k w_k|.  Near-zero
    outputs (cancellation) are judged by the size of their terms, not by the
    ulp of the tiny result."""
    K = x.shape[1]
    # the products in float64 on the GPU (exact to ~1e-16 relative: fp16
    # operands, float64 accumulation)
    x64, w64 = torch.from_numpy(x).cuda().double(), torch.from_numpy(w).cuda().double()
    y = (x64 @ w64.T).cpu().numpy() + (b.astype(np.float64) if epi != "none" else 0.0)
    acc = 4.0 * np.sqrt(K) * 2.0 ** -24 * (x64.abs() @ w64.abs().T).cpu().numpy()
    del x64, w64
    half = 0.5 * np.maximum(ulp16(y), ulp16(out))
    if epi in ("none", "bias"):
        bound, want = half + acc, y
    elif epi == "relu":
        bound, want = half + acc, np.maximum(y, 0)
    else:  # gelu(fp16(y)): |gelu'| <= 1.13, two roundings
        want = O.gelu(y, round16=False)
        bound = 0.5 * np.maximum(ulp16(want), ulp16(out)) + 1.13 * (half + acc)
    err = np.abs(out - want)
    worst = np.argmax(err - bound)
    assert np.all(err <= bound + 1e-12), f"err {err.flat[worst]:.3g} > bound {bound.flat[worst]:.3g}"
    # the common case is exact agreement with the once-rounded reference value
    if epi in ("none", "bias"):
        assert np.mean(out != O.f16(y)) < 5e-3


@pytest.mark.parametrize("epi,n,k", [("bias", 4096, 1024), ("gelu", 4096, 1024), ("bias", 3072, 1024),
                                     ("bias", 1024, 1024), ("bias", 1024, 4096)])
def test_linear_rows_do_not_depend_on_m(epi, n, k):
    """Every GEMM kernel accumulates an element over the same K slices in the
    same order and rounds it the same way: the first rows of an 8192-row
    product (256 x 256 tiles at N = 4096, 256 x 192 at N = 3072, 256-row tiles
    at N = 1024) equal,
    bit for bit, the same rows computed alone (7 and 32 rows: the 32 x 16
    tiles on 16 x 16 x 16 MFMAs; 160 rows: the 64 x 64 tiles; 792 to 3,500:
    the tiles the cost model picks up to 4,096 rows -- at N = 4096 128 x 128,
    160 x 128 or 192 x 128 (GELU), 192 x 128, 256 x 128 and 256 x 256, at N =
    1024 64 x 64, 128 x 128 and 160 x 128; 4896: 320 x 256 tiles with GELU,
    256 x 256 + 128 x 128 without (one round of 256 x 256 at N = 3072, the
    QKV shape), 160 x 128 at N = 1024 (eight waves of three or two row
    groups), also at K = 4096: the FFN-down shape; 5100: the same kernels
    with a last tile row of 140 rows, which ends inside the two-group waves'
    rows of the 160 x 128 tiles)."""
    r = np.random.default_rng(21)
    x = r.standard_normal((8192, k)).astype(np.float16)
    w = (r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16)
    b = r.standard_normal(n).astype(np.float16)
    def bits(t):
        torch.cuda.synchronize()
        return t.cpu().numpy().view(np.uint16)

    full = bits(fk().linear(dev(x), dev(w), dev(b), epilogue=epi))
    for m in (7, 32, 160, 792, 1100, 1500, 1800, 2600, 3500, 4896, 5100):
        np.testing.assert_array_equal(bits(fk().linear(dev(x[:m]), dev(w), dev(b), epilogue=epi)), full[:m])


@pytest.mark.parametrize("m,n", [(7, 256), (32, 256), (300, 256), (4200, 1024)])
def test_linear_strided_operands(m, n):
    """gd_linear with lda > k and ldc > n (the skinny tiles at 7 and 32 rows,
    the 64 x 64 tiles at 300, the eight-wave 160 x 128 tiles at 4,200): the
    padding columns of A are never read into the product and those of C are
    never written."""
    from gliner_decide import _native as N
    from gliner_decide.device import stream_handle
    k, lda, ldc = 256, 320, n + 32
    r = np.random.default_rng(m)
    x = r.standard_normal((m, lda)).astype(np.float16)
    x[:, k:] = np.float16(np.nan)  # read into the product, these would poison it
    w = (r.standard_normal((n, k)) / 16).astype(np.float16)
    b = r.standard_normal(n).astype(np.float16)
    dx, dw, db = dev(x), dev(w), dev(b)
    c = torch.full((m, ldc), 7.0, dtype=torch.float16, device="cuda")
    N.check(N.lib().gd_linear(dx.data_ptr(), dw.data_ptr(), db.data_ptr(), c.data_ptr(), m, n, k, lda, ldc, None, 0,
                              N.GD_EPI_BIAS, stream_handle()))
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    assert np.all(got[:, n:] == np.float16(7.0))
    check_linear(got[:, :n], np.ascontiguousarray(x[:, :k]), w, b, "bias")


def test_linear_row_gather():
    r = np.random.default_rng(8)
    x = r.standard_normal((500, 1024)).astype(np.float16)
    w = (r.standard_normal((2048, 1024)) / 32).astype(np.float16)
    b = r.standard_normal(2048).astype(np.float16)
    rows = r.integers(0, 500, size=77).astype(np.int32)
    out = host(fk().linear(dev(x), dev(w), dev(b), epilogue="relu", rows=dev(rows)))
    check_linear(out, x[rows], w, b, "relu")


def _ordered16(a):
    """fp16 bit patterns mapped to integers that are monotone in the value
    (so a difference of 1 is one ulp, across zero as well)."""
    i = np.asarray(a, np.float16).view(np.int16).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFF), i)


@pytest.mark.parametrize("m,n", [(32, 2048), (248, 256), (2048, 256), (4896, 4096), (8192, 4096)])
def test_gelu_epilogue_every_fp16_input(m, n):
    """x @ I^T + 0 reproduces x exactly, so the GELU epilogue sees every finite
    fp16 value once (63488 = 248 x 256).  Every kernel (the 32 x 16 tiles at
    M = 32, the small-M tiles at M = 248, 256x128 at M = 2048, 320x256 at 4896,
    256x256 at 8192) reads the correctly rounded table: exact everywhere."""
    vals = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    vals = vals[np.isfinite(vals)]
    x = np.zeros((m, n), np.float16)
    x.flat[:vals.size] = vals
    w = np.eye(n, dtype=np.float16)
    b = np.zeros(n, np.float16)
    out = fk().linear(dev(x), dev(w), dev(b), epilogue="gelu")
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(-1)[:vals.size]
    want = O.gelu(vals.astype(np.float64))
    d = np.abs(_ordered16(got) - _ordered16(want))
    assert d.max() == 0, f"{d.max()} ulp at x={vals[np.argmax(d)]}"
    if n == 4096:  # |x| >= 8, infinities and NaN take the table-free branch
        special = np.array([8.0, -8.0, 65504.0, -65504.0, np.inf, -np.inf, np.nan], np.float16)
        x2 = np.zeros((m, n), np.float16)
        diag = np.arange(special.size)
        x2[diag, diag] = special  # one per row: inf * 0 would spread NaN along a row
        out2 = fk().linear(dev(x2), dev(w), dev(b), epilogue="gelu")
        torch.cuda.synchronize()
        got2 = out2.cpu().numpy()[diag, diag]
        np.testing.assert_array_equal(got2[:4].view(np.uint16),
                                      np.array([8.0, -0.0, 65504.0, -0.0], np.float16).view(np.uint16))
        assert got2[4] == np.inf and np.isnan(got2[5]) and np.isnan(got2[6])


# ---------------------------------------------------------------------------
# fused relative bias + masked softmax (+ P.V) -- DeBERTa.swift:322-395
# ---------------------------------------------------------------------------
def _attn_case(seed, B, H, L, min_len=None):
    r = np.random.default_rng(seed)
    D, P = 64, 512
    q = r.standard_normal((B, H, L, D)).astype(np.float16)
    k = r.standard_normal((B, H, L, D)).astype(np.float16)
    v = r.standard_normal((B, H, L, D)).astype(np.float16)
    pk = r.standard_normal((P, H * D)).astype(np.float16)  # [P, H*D] as the projection writes it
    pq = r.standard_normal((P, H * D)).astype(np.float16)
    lengths = r.integers(min_len or max(1, L // 2), L + 1, size=B)
    lengths[0] = L
    mask = (np.arange(L)[None, :] < lengths[:, None]).astype(np.float16)
    return q, k, v, pk, pq, mask


def _tables(pk, pq, H):
    P = pk.shape[0]
    return pk.reshape(P, H, 64).transpose(1, 0, 2), pq.reshape(P, H, 64).transpose(1, 0, 2)


def _oracle_probs(q, k, pk, pq, mask):
    H, L = q.shape[1], q.shape[2]
    pkh, pqh = _tables(pk, pq, H)
    c2p, p2c = O.relative_indices(L)
    bias = O.relative_bias_default(q, k, pkh, pqh, c2p, p2c, 64)
    return bias, O.attention_probs_default(q, k, bias, mask, 64)


def _bias_terms(q, k, pk, pq):
    """The fp16 c2p and p2c terms of the default graph, gathered to [B,H,L,L]."""
    H, L = q.shape[1], q.shape[2]
    pkh, pqh = _tables(pk, pq, H)
    c2p, p2c = O.relative_indices(L)
    c2p_raw = O.f16(np.einsum("bhld,hpd->bhlp", q.astype(np.float64), pkh.astype(np.float64), optimize=True))
    p2c_raw = O.f16(np.einsum("bhld,hpd->bhlp", k.astype(np.float64), pqh.astype(np.float64), optimize=True))
    rows = np.arange(L)[:, None]
    return c2p_raw[:, :, rows, c2p], np.swapaxes(p2c_raw[:, :, rows, p2c], -1, -2)


def _gpu_tables(pk, pq, H):
    tpk, tpq = dev(pk), dev(pq)
    P = pk.shape[0]
    return tpk.view(P, H, 64).permute(1, 0, 2), tpq.view(P, H, 64).permute(1, 0, 2)


@pytest.mark.parametrize("L", [16, 32, 48, 96, 128, 160, 256, 512])
def test_attention_probs_and_bias(L):
    B, H = 2, 3
    q, k, v, pk, pq, mask = _attn_case(L, B, H, L)
    gpk, gpq = _gpu_tables(pk, pq, H)
    bias, probs = _oracle_probs(q, k, pk, pq, mask)
    got = host(fk().deberta_attention(dev(q), dev(k), None, gpk, gpq, dev(mask), output="probs"))
    assert np.max(np.abs(got - probs)) <= 1e-3
    valid = mask[:, None, None, :] > 0
    assert np.all(got[~np.broadcast_to(valid, got.shape)] == 0)  # masked keys get exactly 0
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=3e-3)
    gb = host(fk().deberta_attention(dev(q), dev(k), None, gpk, gpq, dev(mask), output="bias"))
    want_b = O.f16(bias + O.additive_key_mask(mask))
    fin = np.isfinite(want_b)
    np.testing.assert_array_equal(np.isfinite(gb), fin)
    # fp32 (GPU) vs float64 (oracle) accumulation may flip c2p, p2c or their
    # fp16 sum by one ulp; each flip moves the bias by ulp / fp16(sqrt(192)).
    c2p16, p2c16 = _bias_terms(q, k, pk, pq)
    s16 = O.f16(c2p16 + p2c16)
    bound = (ulp16(c2p16) + ulp16(p2c16) + ulp16(s16)) / O.scale_f16(64) + ulp16(bias)
    bound = np.broadcast_to(bound, want_b.shape)
    err = np.abs(gb - want_b)
    assert np.all(err[fin] <= bound[fin]), err[fin].max()
    assert np.mean(err[fin] > 0) < 2e-2


@pytest.mark.parametrize("L", [32, 96, 256, 512])
def test_attention_context(L):
    B, H = 2, 2
    q, k, v, pk, pq, mask = _attn_case(100 + L, B, H, L)
    gpk, gpq = _gpu_tables(pk, pq, H)
    pkh, pqh = _tables(pk, pq, H)
    c2p, p2c = O.relative_indices(L)
    bias = O.relative_bias_default(q, k, pkh, pqh, c2p, p2c, 64)
    want = O.attention_default(q, k, v, bias, mask, 64)
    got = host(fk().deberta_attention(dev(q), dev(k), dev(v), gpk, gpq, dev(mask), output="context"))
    assert got.shape == (B, L, H * 64)
    assert np.max(np.abs(got - want)) <= 4e-3, np.max(np.abs(got - want))


def test_attention_strided_fused_projection_layout():
    """Q, K, V as views of one [B, L, 3, H, D] projection (the encoder's layout)."""
    B, H, L = 2, 4, 128
    r = np.random.default_rng(21)
    qkv = r.standard_normal((B, L, 3, H, 64)).astype(np.float16)
    pk = r.standard_normal((512, H * 64)).astype(np.float16)
    pq = r.standard_normal((512, H * 64)).astype(np.float16)
    mask = np.ones((B, L), np.float16)
    mask[1, 100:] = 0
    t = dev(qkv)
    q, k, v = (t[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    gpk, gpq = _gpu_tables(pk, pq, H)
    got = host(fk().deberta_attention(q, k, v, gpk, gpq, dev(mask), output="context"))
    qn, kn, vn = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    want = host(fk().deberta_attention(dev(qn), dev(kn), dev(vn), gpk, gpq, dev(mask), output="context"))
    np.testing.assert_array_equal(got, want)


def test_attention_full_size_relbias_workload():
    """The relative-bias + masked-softmax workload at its full size (B=32,
    H=16, L=256, D=64, key lengths U[16, 256]): every (b, h) slice of both
    outputs against the oracle, in chunks of 4 batch rows.  Probabilities
    within 1e-3 everywhere, masked keys exactly 0, rows summing to 1; the
    SDPA bias within the propagated one-ulp flips of the fp16 c2p / p2c / sum
    chain, and exactly equal (inf pattern included) past the fp16 range."""
    from gliner_decide.synthetic import relbias_inputs
    d = relbias_inputs(seed=3)
    H = 16
    gpk, gpq = _gpu_tables(d["pos_key"], d["pos_query"], H)
    got = host(fk().deberta_attention(dev(d["q"]), dev(d["k"]), None, gpk, gpq, dev(d["mask"]), output="probs"))
    got_b = host(fk().deberta_attention(dev(d["q"]), dev(d["k"]), None, gpk, gpq, dev(d["mask"]), output="bias"))
    valid = d["mask"][:, None, None, :] > 0
    assert np.all(got[~np.broadcast_to(valid, got.shape)] == 0)
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=3e-3)
    worst_p, flipped, total = 0.0, 0, 0
    for b0 in range(0, 32, 4):
        sl = slice(b0, b0 + 4)
        q, k, m = d["q"][sl], d["k"][sl], d["mask"][sl]
        bias, probs = _oracle_probs(q, k, d["pos_key"], d["pos_query"], m)
        dp = np.abs(got[sl] - probs)
        worst_p = max(worst_p, float(dp.max()))
        assert dp.max() <= 1e-3, (b0, np.unravel_index(dp.argmax(), dp.shape))
        want_b = O.f16(bias + O.additive_key_mask(m))
        fin = np.isfinite(want_b)
        np.testing.assert_array_equal(np.isfinite(got_b[sl]), fin)
        np.testing.assert_array_equal(got_b[sl][~fin], want_b[~fin])
        c2p16, p2c16 = _bias_terms(q, k, d["pos_key"], d["pos_query"])
        s16 = O.f16(c2p16 + p2c16)
        bound = (ulp16(c2p16) + ulp16(p2c16) + ulp16(s16)) / O.scale_f16(64) + ulp16(bias)
        err = np.abs(got_b[sl] - want_b)
        assert np.all(err[fin] <= np.broadcast_to(bound, err.shape)[fin]), (b0, err[fin].max())
        flipped += int((err[fin] > 0).sum())
        total += int(fin.sum())
    assert flipped / total < 2e-2, flipped / total
    print(f"relbias workload: max |dP| {worst_p:.3g}, bias elements off by a flip {flipped / total:.2e}")


def test_attention_rejects_bad_shapes():
    from gliner_decide import GlinerDecideError
    q = torch.zeros((1, 1, 40, 64), dtype=torch.float16, device="cuda")
    t = torch.zeros((1, 512, 64), dtype=torch.float16, device="cuda")
    m = torch.ones((1, 40), dtype=torch.float16, device="cuda")
    with pytest.raises(GlinerDecideError):
        fk().deberta_attention(q, q, q, t, t, m)  # L = 40 is not a multiple of 16


# ---------------------------------------------------------------------------
# FusedKernels general-index API (FusedKernels.swift:83-123, 13-81)
# ---------------------------------------------------------------------------
def test_relative_bias_known_answer(golden):
    g = golden("relbias_known_answer.npz")
    out = host(fk().relative_bias(dev(g["q"], torch.float16), dev(g["k"], torch.float16),
                                  dev(g["pos_key"], torch.float16), dev(g["pos_query"], torch.float16),
                                  dev(g["c2p"]), dev(g["p2c"]), dev(g["key_mask"], torch.float16),
                                  float(g["scale"]), 1, 2, 8, 4, 8))
    assert_within_ulp(out, g["kernel"].astype(np.float16).astype(np.float64), 1.0)


def test_fused_attention_known_answer(golden):
    g = golden("relbias_known_answer.npz")
    out = host(fk().fused_attention(dev(g["q"], torch.float16), dev(g["k"], torch.float16),
                                    dev(g["v"], torch.float16), dev(g["pos_key"], torch.float16),
                                    dev(g["pos_query"], torch.float16), dev(g["c2p"]), dev(g["p2c"]),
                                    dev(g["key_mask"], torch.float16), float(g["scale"]), 1, 2, 8, 4, 8))
    assert_within_ulp(out, g["fused"].astype(np.float16).astype(np.float64), 1.0)


def test_general_index_kernels_vs_oracle_closed_form():
    B, H, L = 2, 2, 64
    q, k, v, pk, pq, mask = _attn_case(55, B, H, L)
    pkh, pqh = _tables(pk, pq, H)
    c2p, p2c = O.relative_indices(L)
    key_mask = np.where(mask > 0, 0.0, -65504.0).astype(np.float16)
    scale = O.scale_f32(64)
    want = O.relative_bias_kernel(q, k, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().relative_bias(dev(q), dev(k), dev(np.ascontiguousarray(pkh)), dev(np.ascontiguousarray(pqh)),
                                  dev(c2p.astype(np.int32)), dev(p2c.astype(np.int32)), dev(key_mask), scale, B, H, L,
                                  64, 512))
    assert_within_ulp(got, want, 1.0)
    want = O.fused_attention_kernel(q, k, v, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().fused_attention(dev(q), dev(k), dev(v), dev(np.ascontiguousarray(pkh)),
                                    dev(np.ascontiguousarray(pqh)), dev(c2p.astype(np.int32)),
                                    dev(p2c.astype(np.int32)), dev(key_mask), scale, B, H, L, 64, 512))
    assert np.max(np.abs(got - want)) <= 2e-3


# ---------------------------------------------------------------------------
# score chains of the classifier flags (DeBERTa.swift:337-409)
# ---------------------------------------------------------------------------
SCORE_FLAGS = {"explicit": dict(fast=False), "kernel_bias": dict(custom_bias=True),
               "kernel_bias_explicit": dict(custom_bias=True, fast=False), "fused": dict(fused=True)}


@pytest.mark.parametrize("L", [32, 96, 256, 512])
@pytest.mark.parametrize("score", sorted(SCORE_FLAGS))
def test_attention_score_chain_context(L, score):
    """Context of each chain against the oracle's attention stage for the
    same flags (B=2, H=2, one padded row).  Bound 4e-3 as the default chain:
    the fp32 (GPU) vs float64 (oracle) accumulation moves an fp16 rounding
    point by one ulp now and then, which moves a probability by ~1e-3
    relative."""
    B, H = 2, 2
    q, k, v, pk, pq, mask = _attn_case(300 + L, B, H, L)
    gpk, gpq = _gpu_tables(pk, pq, H)
    pkh, pqh = _tables(pk, pq, H)
    want = O.attention_stage(q, k, v, pkh, pqh, mask, 64, **SCORE_FLAGS[score])
    got = host(fk().deberta_attention(dev(q), dev(k), dev(v), gpk, gpq, dev(mask), output="context", score=score))
    assert got.shape == (B, L, H * 64)
    err = np.abs(got - want)
    assert err.max() <= 4e-3, err.max()
    assert np.mean(err > 0) < 0.2  # mostly exact agreement with the rounded oracle


@pytest.mark.parametrize("L", [32, 256, 512])
@pytest.mark.parametrize("score", ["explicit", "kernel_bias", "fused"])
def test_attention_score_chain_probs(L, score):
    """Probabilities: masked keys exactly 0, rows sum to 1, |dP| <= 1e-3
    against the oracle's probabilities of the same chain."""
    B, H = 2, 2
    q, k, v, pk, pq, mask = _attn_case(400 + L, B, H, L)
    gpk, gpq = _gpu_tables(pk, pq, H)
    pkh, pqh = _tables(pk, pq, H)
    c2p, p2c = O.relative_indices(L)
    km = np.where(mask > 0, 0.0, -65504.0)
    if score == "explicit":
        bias = O.relative_bias_default(q, k, pkh, pqh, c2p, p2c, 64)
        qk = np.matmul(q.astype(np.float64), np.swapaxes(k, -1, -2).astype(np.float64))
        s = O.f16(O.f16(O.f16(qk) / O.scale_f16(64)) + bias)
        s = np.where(mask[:, None, None, :] > 0, s, -65504.0)
        want = O.f16(O._softmax(s))
    elif score == "kernel_bias":
        bias = O.relative_bias_kernel(q, k, pkh, pqh, c2p, p2c, km, O.scale_f32(64))
        qk = np.matmul(q.astype(np.float64), np.swapaxes(k, -1, -2).astype(np.float64))
        want = O._softmax(qk * O.scale_f32(64) + bias)
    else:
        hh = np.arange(H)[:, None, None]
        c2pt = np.einsum("bhqd,hqkd->bhqk", q.astype(np.float64), pkh.astype(np.float64)[hh, c2p[None]])
        p2ct = np.einsum("bhkd,hqkd->bhqk", k.astype(np.float64), pqh.astype(np.float64)[hh, p2c.T[None]])
        qk = np.matmul(q.astype(np.float64), np.swapaxes(k, -1, -2).astype(np.float64))
        sc = np.where(mask[:, None, None, :] > 0, (qk + c2pt + p2ct) * O.scale_f32(64), -65504.0)
        want = O._softmax(sc)
    got = host(fk().deberta_attention(dev(q), dev(k), None, gpk, gpq, dev(mask), output="probs", score=score))
    valid = np.broadcast_to(mask[:, None, None, :] > 0, got.shape)
    assert np.all(got[~valid] == 0)
    np.testing.assert_allclose(got.sum(-1), 1.0, atol=3e-3)
    assert np.max(np.abs(got - want)) <= 1e-3


@pytest.mark.parametrize("L", [32, 256, 512])
@pytest.mark.parametrize("score", ["default"] + sorted(SCORE_FLAGS))
def test_attention_all_masked_row(L, score):
    """A batch row with no valid key: the reference adds the mask term to
    every score (fp16(bias + -65504) under SDPA, -65504 from the Metal
    kernels and `where`), so its softmax is a degenerate one over every key,
    not zeros.  Context against the oracle's attention stage (bound 4e-3, as
    the other chains); probabilities sum to 1 and, on the default chain,
    match the oracle within 1e-3 (the GPU forms q.k * s + mask in fp32,
    whose grid at 65504 is 2^-8: |dP| <= P * 2^-9)."""
    B, H = 2, 2
    q, k, v, pk, pq, mask = _attn_case(500 + L, B, H, L)
    mask[1] = 0
    gpk, gpq = _gpu_tables(pk, pq, H)
    pkh, pqh = _tables(pk, pq, H)
    flags = SCORE_FLAGS.get(score, {})
    want = O.attention_stage(q, k, v, pkh, pqh, mask, 64, **flags)
    got = host(fk().deberta_attention(dev(q), dev(k), dev(v), gpk, gpq, dev(mask), output="context", score=score))
    assert np.all(np.isfinite(got))
    err = np.abs(got - want)
    assert err.max() <= 4e-3, err.max()
    assert np.abs(got[1]).max() > 0.05  # not the zeros of a softmax over no key
    probs = host(fk().deberta_attention(dev(q), dev(k), None, gpk, gpq, dev(mask), output="probs", score=score))
    np.testing.assert_allclose(probs.sum(-1), 1.0, atol=3e-3)
    valid = np.broadcast_to(mask[:, None, None, :] > 0, probs.shape)
    assert np.all(probs[0][~valid[0]] == 0)  # the row with valid keys keeps exact zeros
    if score == "default":
        _, want_p = _oracle_probs(q, k, pk, pq, mask)
        assert np.max(np.abs(probs - want_p)) <= 1e-3


@pytest.mark.parametrize("L", [32, 160, 256, 512])
def test_relative_bias_closed_form_indices(L):
    """gd_relative_bias with NULL indices (the MFMA kernel-bias chain) against
    the oracle's Metal-kernel restatement on the closed-form indices: one
    fp16 rounding of an fp32 sum, so within one ulp; masked keys exactly
    -65504.  The general-index kernel on the same indices agrees too."""
    B, H = 2, 3
    q, k, v, pk, pq, mask = _attn_case(500 + L, B, H, L)
    pkh, pqh = (np.ascontiguousarray(t) for t in _tables(pk, pq, H))
    c2p, p2c = O.relative_indices(L)
    key_mask = np.where(mask > 0, 0.0, -65504.0).astype(np.float16)
    scale = O.scale_f32(64)
    want = O.relative_bias_kernel(q, k, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().relative_bias(dev(q), dev(k), dev(pkh), dev(pqh), None, None, dev(key_mask), scale, B, H, L, 64,
                                  512))
    masked = np.broadcast_to(mask[:, None, None, :] == 0, got.shape)
    assert np.all(got[masked] == -65504.0)
    # |fp32 sum - exact| <= 4 sqrt(D) 2^-24 sum|terms| (as for the GEMMs), and
    # each side rounds once to fp16 (half an ulp each): near-zero biases (c2p
    # + p2c cancelling) sit on the 2^-24 subnormal grid, where the
    # accumulation term is several ulps
    acc = 4.0 * 8.0 * 2.0 ** -24 * O.relative_bias_kernel(np.abs(q), np.abs(k), np.abs(pkh), np.abs(pqh), c2p, p2c,
                                                            np.zeros_like(key_mask), scale, round16=False)
    valid = ~masked
    err = np.abs(got - want)[valid]
    bound = (np.maximum(ulp16(got), ulp16(want)) + acc)[valid]
    assert np.all(err <= bound + 1e-12), (err - bound).max()
    assert np.mean(err > 0) < 2e-2  # mostly the same fp16 value as the exactly rounded oracle
    general = host(fk().relative_bias(dev(q), dev(k), dev(pkh), dev(pqh), dev(c2p.astype(np.int32)),
                                      dev(p2c.astype(np.int32)), dev(key_mask), scale, B, H, L, 64, 512))
    err = np.abs(got - general)[valid]
    bound = (np.maximum(ulp16(got), ulp16(general)) + 2 * acc)[valid]
    assert np.all(err <= bound + 1e-12), (err - bound).max()


@pytest.mark.parametrize("L", [32, 256, 512])
def test_fused_attention_closed_form_indices(L):
    """gd_fused_attention with NULL indices (the MFMA fused chain) against the
    oracle's restatement of the fused Metal kernel: [B, L, H, D] output."""
    B, H = 2, 2
    q, k, v, pk, pq, mask = _attn_case(600 + L, B, H, L)
    pkh, pqh = (np.ascontiguousarray(t) for t in _tables(pk, pq, H))
    c2p, p2c = O.relative_indices(L)
    key_mask = np.where(mask > 0, 0.0, -65504.0).astype(np.float16)
    scale = O.scale_f32(64)
    want = O.fused_attention_kernel(q, k, v, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().fused_attention(dev(q), dev(k), dev(v), dev(pkh), dev(pqh), None, None, dev(key_mask), scale, B,
                                    H, L, 64, 512))
    assert got.shape == (B, L, H, 64)
    assert np.max(np.abs(got - want)) <= 2e-3


@pytest.mark.parametrize("L,P,H", [(32, 512, 2), (48, 200, 3), (144, 300, 2), (256, 512, 8), (512, 512, 1)])
def test_general_index_kernels_random_indices(L, P, H):
    """gd_relative_bias and gd_fused_attention with arbitrary index tensors
    (the matrix-core kernels: D = 64, L a multiple of 16) against the
    oracle's restatement of the Metal kernels.  Per-head random indices;
    L = 144 leaves a partial key block (one 16-key block) and a query block
    with one active wave, L = 48 three 16-key blocks (a partial group of the
    bias kernel's four-block store transpose) and three active waves, P = 300
    a partial table pass; the last batch row has every key masked (the
    reference's uniform softmax over -65504)."""
    B = 3
    r = np.random.default_rng(900 + L)
    q, k, v = (r.standard_normal((B, H, L, 64)).astype(np.float16) for _ in range(3))
    pkh, pqh = (r.standard_normal((H, P, 64)).astype(np.float16) for _ in range(2))
    c2p = r.integers(0, P, size=(H, L, L)).astype(np.int32)
    p2c = r.integers(0, P, size=(H, L, L)).astype(np.int32)
    lengths = np.array([L, max(1, L // 3), 0])
    key_mask = np.where(np.arange(L)[None, :] < lengths[:, None], 0.0, -65504.0).astype(np.float16)
    scale = O.scale_f32(64)
    want = O.relative_bias_kernel(q, k, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().relative_bias(dev(q), dev(k), dev(pkh), dev(pqh), dev(c2p), dev(p2c), dev(key_mask), scale, B, H,
                                  L, 64, P))
    masked = np.broadcast_to(key_mask[:, None, None, :] < -60000, got.shape)
    assert np.all(got[masked] == -65504.0)
    acc = 4.0 * 8.0 * 2.0 ** -24 * O.relative_bias_kernel(np.abs(q), np.abs(k), np.abs(pkh), np.abs(pqh), c2p, p2c,
                                                            np.zeros_like(key_mask), scale, round16=False)
    err = np.abs(got - want)[~masked]
    bound = (np.maximum(ulp16(got), ulp16(want)) + acc)[~masked]
    assert np.all(err <= bound + 1e-12), (err - bound).max()
    want = O.fused_attention_kernel(q, k, v, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().fused_attention(dev(q), dev(k), dev(v), dev(pkh), dev(pqh), dev(c2p), dev(p2c), dev(key_mask),
                                    scale, B, H, L, 64, P))
    assert got.shape == (B, L, H, 64)
    assert np.max(np.abs(got - want)) <= 2e-3
    # the fully masked row: the plain mean of V over every key
    np.testing.assert_allclose(got[2], np.broadcast_to(v[2].astype(np.float64).mean(axis=1)[None], (L, H, 64)),
                               atol=2e-3)


def test_general_index_kernels_clamp_out_of_range_indices():
    """Indices outside [0, P) read the nearest table row (the per-query
    kernels' rule, kept by the matrix-core kernels)."""
    B, H, L, P = 2, 2, 64, 200
    r = np.random.default_rng(77)
    q, k, v = (r.standard_normal((B, H, L, 64)).astype(np.float16) for _ in range(3))
    pkh, pqh = (r.standard_normal((H, P, 64)).astype(np.float16) for _ in range(2))
    c2p = r.integers(-40, P + 40, size=(H, L, L)).astype(np.int32)
    p2c = r.integers(-40, P + 40, size=(H, L, L)).astype(np.int32)
    key_mask = np.zeros((B, L), np.float16)
    scale = O.scale_f32(64)
    c2pc, p2cc = np.clip(c2p, 0, P - 1), np.clip(p2c, 0, P - 1)
    want = O.relative_bias_kernel(q, k, pkh, pqh, c2pc, p2cc, key_mask, scale)
    got = host(fk().relative_bias(dev(q), dev(k), dev(pkh), dev(pqh), dev(c2p), dev(p2c), dev(key_mask), scale, B, H,
                                  L, 64, P))
    acc = 4.0 * 8.0 * 2.0 ** -24 * O.relative_bias_kernel(np.abs(q), np.abs(k), np.abs(pkh), np.abs(pqh), c2pc, p2cc,
                                                            key_mask, scale, round16=False)
    assert np.all(np.abs(got - want) <= np.maximum(ulp16(got), ulp16(want)) + acc + 1e-12)
    want = O.fused_attention_kernel(q, k, v, pkh, pqh, c2pc, p2cc, key_mask, scale)
    got = host(fk().fused_attention(dev(q), dev(k), dev(v), dev(pkh), dev(pqh), dev(c2p), dev(p2c), dev(key_mask),
                                    scale, B, H, L, 64, P))
    assert np.max(np.abs(got - want)) <= 2e-3


@pytest.mark.parametrize("L,P", [(16, 512), (32, 65536), (32, 65537)])
def test_general_index_kernels_size_limits(L, P):
    """The shortest sequence (one 16-key block, one active wave), the largest
    table the matrix-core kernels' 16-bit packed indices address (P = 65536,
    indices up to 65535) and one row more (the per-query kernels)."""
    B, H = 2, 1
    r = np.random.default_rng(P + L)
    q, k, v = (r.standard_normal((B, H, L, 64)).astype(np.float16) for _ in range(3))
    pkh, pqh = (r.standard_normal((H, P, 64)).astype(np.float16) for _ in range(2))
    c2p = r.integers(0, P, size=(H, L, L)).astype(np.int32)
    p2c = r.integers(0, P, size=(H, L, L)).astype(np.int32)
    c2p[0, 0, :2] = [0, P - 1]  # both ends of the table
    p2c[0, :2, 0] = [P - 1, 0]
    key_mask = np.zeros((B, L), np.float16)
    key_mask[1, L // 2:] = -65504.0
    scale = O.scale_f32(64)
    want = O.relative_bias_kernel(q, k, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().relative_bias(dev(q), dev(k), dev(pkh), dev(pqh), dev(c2p), dev(p2c), dev(key_mask), scale, B, H,
                                  L, 64, P))
    acc = 4.0 * 8.0 * 2.0 ** -24 * O.relative_bias_kernel(np.abs(q), np.abs(k), np.abs(pkh), np.abs(pqh), c2p, p2c,
                                                            np.zeros_like(key_mask), scale, round16=False)
    assert np.all(np.abs(got - want) <= np.maximum(ulp16(got), ulp16(want)) + acc + 1e-12)
    want = O.fused_attention_kernel(q, k, v, pkh, pqh, c2p, p2c, key_mask, scale)
    got = host(fk().fused_attention(dev(q), dev(k), dev(v), dev(pkh), dev(pqh), dev(c2p), dev(p2c), dev(key_mask),
                                    scale, B, H, L, 64, P))
    assert np.max(np.abs(got - want)) <= 2e-3


def test_general_index_kernels_misaligned_indices():
    """Index tensors 4 bytes off a 16-byte boundary take the per-query
    kernels (the matrix-core kernels read indices four at a time): same
    results as the aligned call, to the oracle's bounds."""
    B, H, L, P = 1, 2, 32, 512
    r = np.random.default_rng(78)
    q, k, v = (r.standard_normal((B, H, L, 64)).astype(np.float16) for _ in range(3))
    pkh, pqh = (r.standard_normal((H, P, 64)).astype(np.float16) for _ in range(2))
    c2p = r.integers(0, P, size=(H, L, L)).astype(np.int32)
    p2c = r.integers(0, P, size=(H, L, L)).astype(np.int32)
    key_mask = np.zeros((B, L), np.float16)
    key_mask[0, -3:] = -65504.0
    scale = O.scale_f32(64)

    def off4(a):  # the same values starting 4 bytes into a 16-byte aligned allocation
        buf = torch.empty(a.size + 1, dtype=torch.int32, device="cuda")
        buf[1:] = torch.from_numpy(a.reshape(-1)).cuda()
        t = buf[1:].view(a.shape)
        assert t.data_ptr() % 16 == 4
        return t

    want = O.relative_bias_kernel(q, k, pkh, pqh, c2p, p2c, key_mask, scale)
    acc = 4.0 * 8.0 * 2.0 ** -24 * O.relative_bias_kernel(np.abs(q), np.abs(k), np.abs(pkh), np.abs(pqh), c2p, p2c,
                                                            np.zeros_like(key_mask), scale, round16=False)
    for c, p in ((dev(c2p), dev(p2c)), (off4(c2p), off4(p2c))):
        got = host(fk().relative_bias(dev(q), dev(k), dev(pkh), dev(pqh), c, p, dev(key_mask), scale, B, H, L, 64, P))
        assert np.all(np.abs(got - want) <= np.maximum(ulp16(got), ulp16(want)) + acc + 1e-12)
    want = O.fused_attention_kernel(q, k, v, pkh, pqh, c2p, p2c, key_mask, scale)
    for c, p in ((dev(c2p), dev(p2c)), (off4(c2p), off4(p2c))):
        got = host(fk().fused_attention(dev(q), dev(k), dev(v), dev(pkh), dev(pqh), c, p, dev(key_mask), scale, B,
                                        H, L, 64, P))
        assert np.max(np.abs(got - want)) <= 2e-3


def test_attention_rejects_bias_output_on_chains_without_a_bias():
    from gliner_decide import GlinerDecideError
    q, k, v, pk, pq, mask = _attn_case(7, 1, 1, 32)
    gpk, gpq = _gpu_tables(pk, pq, 1)
    for score in ("explicit", "kernel_bias_explicit", "fused"):
        with pytest.raises(GlinerDecideError):
            fk().deberta_attention(dev(q), dev(k), dev(v), gpk, gpq, dev(mask), output="bias", score=score)


def test_mfma_forms_agree_bit_for_bit():
    """The GEMM for at most 32 rows runs v_mfma_f32_16x16x16_f16, the tile
    kernels v_mfma_f32_32x32x16_f16; a row's bits do not depend on M only if
    both forms give the same fp32 result for the same 16 products and
    accumulator.  Checked over normal operands, exponents spread over 2^+-12,
    pairs of products that cancel to a few ulps, and accumulators far larger
    than the products; the 32 x 32 form is also held to the fp64 value within
    the fp32 summation bound (so a wrong operand layout in either form
    fails)."""
    from gliner_decide import _native as N
    from gliner_decide.device import stream_handle
    r = np.random.default_rng(17)
    T = 2048
    a = r.standard_normal((T, 32, 16))
    w = r.standard_normal((T, 32, 16))
    c0 = r.standard_normal((T, 32, 32))
    kind = np.arange(T) % 4
    wide = kind == 1
    a[wide] *= np.exp2(r.integers(-12, 13, size=a[wide].shape))
    w[wide] *= np.exp2(r.integers(-12, 13, size=w[wide].shape))
    c0[wide] *= np.exp2(r.integers(-12, 13, size=c0[wide].shape))
    cancel = kind == 2  # product k + 8 = -(product k) (1 + ~2^-9): the slice sums to a few ulps
    a[cancel, :, 8:] = -a[cancel, :, :8] * (1 + np.exp2(-9) * r.standard_normal((cancel.sum(), 32, 8)))
    w[cancel, :, 8:] = w[cancel, :, :8]
    c0[kind == 3] *= 2.0 ** 14
    a16, w16, c32 = a.astype(np.float16), w.astype(np.float16), c0.astype(np.float32)
    da, dw, dc = dev(a16), dev(w16), dev(c32)
    d32 = torch.empty((T, 32, 32), dtype=torch.float32, device="cuda")
    d16 = torch.empty_like(d32)
    N.check(N.lib().gd_diag_mfma_forms(da.data_ptr(), dw.data_ptr(), dc.data_ptr(), d32.data_ptr(), d16.data_ptr(),
                                       T, stream_handle()))
    torch.cuda.synchronize()
    g32, g16 = d32.cpu().numpy(), d16.cpu().numpy()
    np.testing.assert_array_equal(g32.view(np.uint32), g16.view(np.uint32))
    exact = np.einsum("tik,tjk->tij", a16.astype(np.float64), w16.astype(np.float64)) + c32.astype(np.float64)
    scale = np.einsum("tik,tjk->tij", np.abs(a16.astype(np.float64)), np.abs(w16.astype(np.float64))) + np.abs(c32)
    # (an fp32 sum of 17 terms: at most 17 roundings of 2^-24 relative; a
    # wrong operand layout is off by the size of the terms)
    err = np.abs(g32 - exact) / scale
    print(f"mfma forms: max error {err.max() * 2.0 ** 24:.2f} units of 2^-24 of the terms' sum")
    assert err.max() <= 17 * 2.0 ** -24


def test_stream_probe_adds():
    """The streaming-ceiling diagnostic computes what it claims (c = a + b,
    fp16), including a tail shorter than one block."""
    from gliner_decide import _native as N
    from gliner_decide.device import stream_handle
    for n in (8192 * 1024, 32 * 37):
        a = torch.randn(n, device="cuda").half()
        b = torch.randn(n, device="cuda").half()
        c = torch.empty_like(a)
        N.check(N.lib().gd_stream_probe_add(a.data_ptr(), b.data_ptr(), c.data_ptr(), n, stream_handle()))
        torch.cuda.synchronize()
        assert torch.equal(c, a + b)
