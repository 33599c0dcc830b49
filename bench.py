"""Benchmark: 24-layer DeBERTa-v3-large encoder + GLiNER classifier head on one
MI355X, B=32 rows of L=256 tokens per step (synthetic seeded inputs and
random-init fp16 weights of the real architecture).

One step = one `classify` of a 32-row batch (embedding, 24 layers, classifier)
with inputs resident in HBM, ending with the logits copied to pinned host
memory.  Prints ONE JSON line on stdout (logs on stderr): rows/s over exactly
--steps timed steps, the roofline of the dominant kernel (measured live with
HIP events on the launch stream, first thing in the process after a warm-up
of the same launches: the launch sequence of `--profile-kernel`, whose
rocprofv3 summary is committed under profiles/), a CPU baseline (the batched torch fp32
restatement of the reference graph on this host's cores), the single layer at
B=1 L=32 and the long-context batch (B=64, L=512).

Kernel timings use rotating buffer sets larger than the 256 MB Infinity Cache
so that HBM, not the cache, serves the reads, and time each kernel after
0.1 s (at most 2000 launches) of its own launches (the clocks of an idle GPU
ramp up under load).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "gliner-decide-metal_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
# FFN-up + GELU: the single product with the largest share of the step
# (24.3% in profiles/e2e_classify_b32_l256.md; out-proj and FFN-down together
# take 30.6% through one kernel, each less than FFN-up)
ROOFLINE_KERNEL = "ffn_up_gelu"
FP16_DENSE_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
ROTATE_BYTES = 600 << 20  # > 2x the 256 MB MALL


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="classify", choices=["classify", "long_context"])
    p.add_argument("--compiled", action="store_true", help="replay a captured hipGraph per step")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-bucket-mix", action="store_true", help="skip the mixed-length throughput field")
    p.add_argument("--bucket-mix", action="store_true",
                   help="only the mixed-length workload (4096 rows over the L32..L512 buckets), its own JSON line")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--kernel-iters", type=int, default=60)
    p.add_argument("--profile-kernel", default=None,
                   choices=["residual_layernorm", "stream_ceiling", "relbias_softmax", "relative_bias", "attention_context", "qkv_proj",
                            "out_proj", "ffn_up_gelu", "ffn_down", "general_relative_bias",
                            "general_fused_attention"],
                   help="only run this kernel (--kernel-iters launches on rotating buffers) followed by a 256 MiB "
                        "torch copy, for rocprofv3 counter runs; prints the kernel table, no JSON line")
    p.add_argument("--profile-layer", action="store_true",
                   help="only time one encoder layer at B=1, L=32 (gd_classifier_layer_forward, 200 calls after 10 "
                        "untimed, a one-layer model of the same shapes), for rocprofv3 kernel traces; prints its "
                        "time, no JSON line")
    p.add_argument("--serving", action="store_true",
                   help="time the JSONL runner instead (4096 text examples: JSON parse, schema formatting and "
                        "tokenization, H2D, forward, D2H, decode) and print its own JSON line")
    return p.parse_args()


# ---------------------------------------------------------------------------
# live kernel timing
# ---------------------------------------------------------------------------
def gemm_tile(M, N, gelu=False, cus=256):
    """The tile launch_linear picks above 4,096 rows (gemm.hip): one round
    of 320x256 (GELU) or 160x128 (eight waves, no GELU) tiles where it fits,
    whole rounds of 256x256 plus a 128x128 remainder where the remainder
    would cost the 256x256 launch a further round, or the fewest rounds of
    tiles weighted by their relative cost."""
    def rounds(bm, bn):
        return -(-(-(-M // bm) * (N // bn)) // cus)
    if N % 256 == 0:
        per_round = cus // (N // 256)
        if gelu and per_round * 256 < M <= per_round * 320:
            return "320,256"
        full = M // (per_round * 256) * (per_round * 256) if per_round else 0
        rest = M - full
        if full > 0 and rest > 0 and (rest + 127) // 128 * (N // 128) <= cus:
            def rounds256(rows):
                return -(-(-(-rows // 256) * (N // 256)) // cus)
            if rounds256(full) < rounds256(M):
                return "256,256 + 128,128"
    if not gelu and -(-M // 160) * (N // 128) <= cus:
        return "160,128"
    tile, best = "256,128", rounds(256, 128)
    if rounds(192, 128) * 0.8 < best:
        tile, best = "192,128", rounds(192, 128) * 0.8
    if N % 192 == 0 and rounds(256, 192) * 1.35 <= best:
        tile, best = "256,192", rounds(256, 192) * 1.35
    if N % 256 == 0 and rounds(256, 256) * 1.5 <= best:
        tile, best = "256,256", rounds(256, 256) * 1.5
    if gelu and N % 256 == 0 and rounds(320, 256) * 1.95 < best:
        tile = "320,256"
    return tile


WARM_S, WARM_MAX = 0.1, 2000  # untimed launches before a kernel is timed: 0.1 s, at most 2000


def time_launches(fn, sets, iters, warm_s=WARM_S):
    """Average duration (us) of fn(set) over `iters` launches cycling through
    the buffer sets, between two events on the launch stream, after `warm_s`
    seconds (at most WARM_MAX launches) of the same launches untimed: the
    GPU's clocks ramp up under load
    (FFN-up at 8192 rows: 87.7 us over its first 60 launches from idle,
    78.5-79 us sustained, 93 us after 2 s idle), so the timed launches run at
    the clocks a busy GPU holds.  The warm-up synchronises every 32 launches,
    so its wall time follows the GPU's."""
    import torch
    i, t_end = 0, time.perf_counter() + warm_s
    while i < 2 or (time.perf_counter() < t_end and i < WARM_MAX):
        fn(sets[i % len(sets)])
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(sets[i % len(sets)])
    end.record()
    end.synchronize()
    return start.elapsed_time(end) * 1000.0 / iters


def measure_kernels(model_cfg, iters, only=None):
    """Times each kernel of the step at the workload's shapes (or just `only`)."""
    import torch
    from gliner_decide import _native as N
    from gliner_decide.device import stream_handle
    from gliner_decide.fused_kernels import FusedKernels
    from gliner_decide.synthetic import normal16, relbias_inputs
    import math
    import numpy as np

    fk = FusedKernels()
    lib = N.lib()
    dev = torch.device("cuda")
    out = {}
    want = (lambda name: only is None or only == name)

    # residual-add LayerNorm, 8192 x 1024 (the model's shape at B=32, L=256)
    if want("residual_layernorm"):
        rows, cols = 8192, 1024
        nbytes = 3 * rows * cols * 2 + 2 * cols * 2
        nsets = max(2, ROTATE_BYTES // (3 * rows * cols * 2) + 1)
        g = torch.from_numpy(normal16(2, "gamma", (cols,), 1.0, 0.1)).to(dev)
        b = torch.from_numpy(normal16(2, "beta", (cols,), 0.0, 0.1)).to(dev)
        x0 = torch.from_numpy(normal16(2, "x", (rows, cols))).to(dev)
        r0 = torch.from_numpy(normal16(2, "residual", (rows, cols))).to(dev)
        sets = [(x0.roll(i, 0).contiguous(), r0.roll(i, 0).contiguous(), torch.empty_like(x0)) for i in range(nsets)]

        def ln(s):
            N.check(lib.gd_residual_layer_norm(s[0].data_ptr(), s[1].data_ptr(), g.data_ptr(), b.data_ptr(),
                                               s[2].data_ptr(), rows, cols, 1e-7, N.GD_LN_SUM_F16, stream_handle()))

        us = time_launches(ln, sets, iters)
        out["residual_layernorm"] = dict(kernel="residual_ln_kernel<2>", shape=[rows, cols], us=us, bytes=nbytes,
                                         gbs=nbytes / us / 1e3, bound="hbm", launches_per_step=48)
        del sets

    # the same bytes with no arithmetic: two 16-byte non-temporal reads and one
    # write per piece (gd_stream_probe_add), the streaming ceiling of the LN's
    # access pattern on this device
    if want("stream_ceiling"):
        rows, cols = 8192, 1024
        nsets = max(2, ROTATE_BYTES // (3 * rows * cols * 2) + 1)
        sets = [(torch.randn(rows, cols, device=dev).half(), torch.randn(rows, cols, device=dev).half(),
                 torch.empty((rows, cols), device=dev, dtype=torch.float16)) for _ in range(nsets)]

        def probe(s):
            N.check(lib.gd_stream_probe_add(s[0].data_ptr(), s[1].data_ptr(), s[2].data_ptr(), rows * cols,
                                            stream_handle()))

        us = time_launches(probe, sets, iters)
        nbytes = 3 * rows * cols * 2
        out["stream_ceiling"] = dict(kernel="stream_probe_kernel", shape=[rows, cols], us=us, bytes=nbytes,
                                     gbs=nbytes / us / 1e3, bound="hbm", launches_per_step=0)
        del sets

    # relative bias + masked softmax, B=32 H=16 L=256 D=64 -> P [32,16,256,256]
    B, H, L, D = 32, 16, 256, 64
    d = relbias_inputs(seed=3)
    pk = torch.from_numpy(d["pos_key"]).to(dev).view(512, H, D).permute(1, 0, 2)
    pq = torch.from_numpy(d["pos_query"]).to(dev).view(512, H, D).permute(1, 0, 2)
    mask = torch.from_numpy(d["mask"]).to(dev)
    if want("relbias_softmax"):
        q0 = torch.from_numpy(d["q"]).to(dev)
        k0 = torch.from_numpy(d["k"]).to(dev)
        per_set = (2 * B * H * L * D + B * H * L * L) * 2
        nsets = max(2, ROTATE_BYTES // per_set + 1)
        sets = [(q0.roll(i, 0).contiguous(), k0.roll(i, 0).contiguous(),
                 torch.empty((B, H, L, L), dtype=torch.float16, device=dev)) for i in range(nsets)]
        nbytes = 2 * B * H * L * D * 2 + 2 * 512 * H * D * 2 + B * 4 + B * H * L * L * 2

        def rb(s):
            fk.deberta_attention(s[0], s[1], None, pk, pq, mask, output="probs", out=s[2])

        us = time_launches(rb, sets, iters)
        out["relbias_softmax"] = dict(kernel="deberta_attention_kernel<16,PROBS>", shape=[B, H, L, L], us=us,
                                      bytes=nbytes, gbs=nbytes / us / 1e3, bound="hbm", launches_per_step=0)
        del sets

    # the relative-position bias alone (the reference's relativeBias kernel):
    # fp16 bias with masked keys at -65504, [32,16,256,256]
    if want("relative_bias"):
        q0 = torch.from_numpy(d["q"]).to(dev)
        k0 = torch.from_numpy(d["k"]).to(dev)
        per_set = (2 * B * H * L * D + B * H * L * L) * 2
        nsets = max(2, ROTATE_BYTES // per_set + 1)
        sets = [(q0.roll(i, 0).contiguous(), k0.roll(i, 0).contiguous(),
                 torch.empty((B, H, L, L), dtype=torch.float16, device=dev)) for i in range(nsets)]
        nbytes = 2 * B * H * L * D * 2 + 2 * 512 * H * D * 2 + B * L * 2 + B * H * L * L * 2

        def rbias(s):
            fk.deberta_attention(s[0], s[1], None, pk, pq, mask, output="bias", out=s[2])

        us = time_launches(rbias, sets, iters)
        out["relative_bias"] = dict(kernel="deberta_attention_kernel<16,BIAS>", shape=[B, H, L, L], us=us,
                                    bytes=nbytes, gbs=nbytes / us / 1e3, bound="hbm", launches_per_step=0)
        del sets

    # the FusedKernels entry points with index tensors (any indices; here the
    # unbucketed relative positions clip(q - k, -256, 255) + 256 of every head),
    # B=32 H=16 L=256 P=512: the bias [B,H,L,L], and the whole attention [B,L,H,D]
    if want("general_relative_bias") or want("general_fused_attention"):
        P = 512
        r = torch.arange(L)
        rel = ((r[:, None] - r[None, :]).clamp(-256, 255) + 256).int()
        c2p = rel.unsqueeze(0).expand(H, L, L).contiguous().to(dev)
        p2c = rel.t().unsqueeze(0).expand(H, L, L).contiguous().to(dev)
        pkh, pqh = pk.contiguous(), pq.contiguous()
        km = torch.from_numpy(np.where(d["mask"] > 0, 0.0, -65504.0).astype(np.float16)).to(dev)
        q0 = torch.from_numpy(d["q"]).to(dev)
        k0 = torch.from_numpy(d["k"]).to(dev)
        v0 = torch.from_numpy(d["k"][::-1].copy()).to(dev)
        scale = 1.0 / math.sqrt(3 * D)
        common = 2 * H * P * D * 2 + 2 * H * L * L * 4 + B * L * 2
        if want("general_relative_bias"):
            us = time_launches(lambda s: fk.relative_bias(q0, k0, pkh, pqh, c2p, p2c, km, scale, B, H, L, D, P), [0],
                               iters)
            nbytes = 2 * B * H * L * D * 2 + common + B * H * L * L * 2
            out["general_relative_bias"] = dict(kernel="general_mfma_kernel<false>", shape=[B, H, L, L], us=us,
                                                bytes=nbytes, gbs=nbytes / us / 1e3, bound="hbm", launches_per_step=0)
        if want("general_fused_attention"):
            us = time_launches(lambda s: fk.fused_attention(q0, k0, v0, pkh, pqh, c2p, p2c, km, scale, B, H, L, D, P),
                               [0], iters)
            nbytes = 3 * B * H * L * D * 2 + common + B * L * H * D * 2
            out["general_fused_attention"] = dict(kernel="general_mfma_kernel<true>", shape=[B, H, L, D], us=us,
                                                  bytes=nbytes, gbs=nbytes / us / 1e3, bound="hbm",
                                                  launches_per_step=0)
        del c2p, p2c, q0, k0, v0

    # attention as the encoder runs it: context output from the fused QKV layout
    T = B * L
    if want("attention_context"):
        qkv = torch.randn((T, 3 * H * D), device=dev, dtype=torch.float16)
        ctx = torch.empty((T, H * D), device=dev, dtype=torch.float16)
        v5 = qkv.view(B, L, 3, H, D)
        qv, kv_, vv = (v5[:, :, i].permute(0, 2, 1, 3) for i in range(3))
        us = time_launches(lambda s: fk.deberta_attention(qv, kv_, vv, pk, pq, mask, output="context", out=ctx),
                           [0], iters)
        # Roofline: 4 T H D fp16 (Q, K, V in, context out) = 67 MB takes 8.4 us at
        # 8 TB/s, longer than the 17.2 GFLOP (QK^T, c2p, p2c, PV as direct dot
        # products) take at 2.5 PFLOP/s (6.9 us): bounded by HBM.
        flops = 4 * (2 * B * H * L * L * D)
        nbytes = (4 * T * H * D) * 2
        out["attention_context"] = dict(kernel="deberta_attention_kernel<16,CONTEXT>", shape=[B, H, L, D], us=us,
                                        flops=flops, bytes=nbytes, gbs=nbytes / us / 1e3, bound="hbm",
                                        launches_per_step=24, tflops=flops / us / 1e6)
        del qkv, ctx

    # the four projections at T = 8192
    C, F = 1024, 4096
    for name, (n, k, epi) in {"qkv_proj": (3 * C, C, "bias"), "out_proj": (C, C, "bias"),
                              "ffn_up_gelu": (F, C, "gelu"), "ffn_down": (C, F, "bias")}.items():
        if not want(name):
            continue
        a = torch.randn((T, k), device=dev, dtype=torch.float16)
        w = torch.randn((n, k), device=dev, dtype=torch.float16) * 0.02
        bias = torch.randn((n,), device=dev, dtype=torch.float16)
        c = torch.empty((T, n), device=dev, dtype=torch.float16)

        def lin(s, a=a, w=w, bias=bias, c=c, n=n, k=k, epi=epi):
            N.check(lib.gd_linear(a.data_ptr(), w.data_ptr(), bias.data_ptr(), c.data_ptr(), T, n, k, k, n, None, 0,
                                  {"bias": N.GD_EPI_BIAS, "gelu": N.GD_EPI_BIAS_GELU}[epi], stream_handle()))

        us = time_launches(lin, [0], iters)
        flops = 2 * T * n * k
        tile = gemm_tile(T, n, epi == 'gelu')
        kname = "gemm_lds_split160_kernel" if tile == "160,128" else f"gemm_nt_lds_kernel<{tile}>"
        out[name] = dict(kernel=kname, shape=[T, n, k], us=us, flops=flops,
                         tflops=flops / us / 1e6, bound="mfma", launches_per_step=24,
                         bytes=(T * k + n * k + T * n) * 2)
        del a, w, c
    torch.cuda.synchronize()
    return out


def bucket_mix_rate(model, passes=2):
    """Rows/s over the mixed-length workload (4096 rows, lengths exp(U(ln 8,
    ln 512)) in buckets L32..L512, B=32 per bucket with the last batch padded
    by copies of its last row, 1-2 tasks x 2-10 labels).  Counts valid rows
    only, as the reference's batch driver does; one untimed pass first so every
    shape's workspace exists."""
    import torch
    from gliner_decide import DecisionInput
    from gliner_decide.decode import row_extents
    from gliner_decide.synthetic import bucket_mix
    batches = []
    for x in bucket_mix(seed=5):
        a = x.arrays()
        ids, mask, mk, mm = DecisionInput(**a).to_device()
        out = torch.empty((ids.shape[0], mk.shape[1], mk.shape[2]), dtype=torch.float16, device=ids.device)
        batches.append((ids, mask, mk, mm, out, x.valid_rows, a))
    rows = sum(b[5] for b in batches)

    def one_pass():
        for ids, mask, mk, mm, out, _, a in batches:
            total = int(row_extents(a["attention_mask"], a["marker_indices"], a["marker_mask"]).sum())
            model.classify_device(ids, mask, mk, mm, out, total_tokens=total)

    one_pass()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(passes):
        one_pass()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert all(torch.isfinite(b[4].float()).all() for b in batches)
    return dict(value=round(rows * passes / elapsed, 1), unit="rows/s", rows=rows, batches=len(batches),
                passes=passes, sample="bucket mix: 4096 rows over L32..L512, B=32 batches, inputs in HBM, "
                                      "packed rows")


def serving_rate(weights, cfg, passes=2):
    """Rows/s of the JSONL runner (RawCLI.swift:104-171) from JSONL text to
    decoded predictions, with the compiled-graph classifier the runner uses:
    JSON parse, schema formatting and tokenization, H2D, forward, D2H and
    decode, batches of 32.  Rows grouped by length (the runner's default) and,
    for comparison, by (L, Hh, O) as the reference groups them.  One untimed
    pass of each captures every shape's graph; each timed pass starts from an
    empty tokenizer cache."""
    import json as _json
    import torch
    from gliner_decide import GLiNERDecideClassifier
    from gliner_decide import raw_cli
    from gliner_decide.synthetic import serving_examples, word_level_frontend
    model = GLiNERDecideClassifier(weights, cfg, use_compiled_graph=True)
    fe = word_level_frontend()
    lines = [_json.dumps(e) for e in serving_examples()]

    def once(by_length):
        fe.clear_cache()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        res = raw_cli.run_examples(raw_cli.iter_jsonl(lines), fe, model, total=len(lines),
                                   group_by_length=by_length)
        wall = time.perf_counter() - t0
        return wall, sum(r["inferenceMilliseconds"] for r in res) / 1e3, \
            sum(r["preprocessingMilliseconds"] for r in res) / 1e3

    out = {}
    for by_length in (True, False):
        once(by_length)
        wall, gpu_s, tok_s = min(once(by_length) for _ in range(passes))
        out["length" if by_length else "shape"] = dict(rows_s=round(len(lines) / wall, 1), wall_s=round(wall, 4),
                                                         gpu_forward_s=round(gpu_s, 4), tokenize_s=round(tok_s, 4))
    return dict(value=out["length"]["rows_s"], unit="rows/s", rows=len(lines), passes=passes,
                grouped_by_length=out["length"], grouped_by_shape=out["shape"],
                sample="4096 JSONL text examples (token counts exp(U(ln 8, ln 512)), 1-2 tasks x 2-10 labels), "
                       "synthetic word-level tokenizer in the C++ front end, batches of 32, compiled graphs")


def calibration_copy(nbytes=256 << 20):
    """A plain device copy of known size: rocprofv3 FETCH_SIZE / WRITE_SIZE of
    this dispatch calibrate the counters against bytes actually moved."""
    import torch
    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    return nbytes


def roofline_of(name, best, iters):
    """Roofline object of kernel `name` from its live measurement `best`."""
    if best["bound"] == "hbm":
        ach, peak, unit = best["gbs"], HBM_PEAK_GBS, "GB/s"
    else:
        ach, peak, unit = best["tflops"], FP16_DENSE_TFLOPS, "TFLOP/s"
    traffic, source = profiled_traffic(name)
    return dict(kernel=name, bound=best["bound"], achieved=round(ach, 2), peak=peak, unit=unit,
                frac=round(ach / peak, 4), traffic=traffic, traffic_source=source, avg_us=round(best["us"], 2),
                launches=iters, measured="first in the process after a warm-up of the same launches, the launch "
                                        f"sequence of `bench.py --profile-kernel {name} --kernel-iters {iters}`",
                algorithmic_per_launch=best["bytes"] if best["bound"] == "hbm" else best["flops"])


def profiled_traffic(kernel):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary of this kernel (profiles/<kernel>.md), counters calibrated with a
    256 MiB copy; None when no summary exists."""
    path = ROOT / "profiles" / f"{kernel}.md"
    if not path.exists():
        return None, None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1]), str(path.relative_to(ROOT))
    return None, None


# ---------------------------------------------------------------------------
# CPU baseline: the batched torch fp32 restatement of the reference graph
# ---------------------------------------------------------------------------
def cpu_baseline(weights, cfg, batch, budget_s, gpu_logits=None):
    """Whole B=32 L=256 batches through oracle/torch_cpu.py (the default
    reference graph in fp32, every row at the full bucket length) on this
    host's cores (OMP_NUM_THREADS, else all), until `budget_s` is spent (at
    least one batch), after a 2-row warm-up."""
    import numpy as np
    import torch
    from oracle import deberta as O
    from oracle.torch_cpu import TorchCPUModel, cpu_description
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    oc = O.Config(**{k: getattr(cfg, k) for k in O.Config.__dataclass_fields__})
    m = TorchCPUModel(weights, oc)
    a = batch.arrays()
    args = [a["input_ids"], a["attention_mask"], a["marker_indices"], a["marker_mask"]]
    m.forward(*[x[:2] for x in args])
    B = a["input_ids"].shape[0]
    done, t0 = 0, time.perf_counter()
    while True:
        logits = m.forward(*args)
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    el = time.perf_counter() - t0
    out = dict(value=round(B * done / el, 3), unit="rows/s", cores=torch.get_num_threads(), kind="port",
               cpu=cpu_description(), backend=f"torch {torch.__version__} CPU, fp32",
               sample=f"{done} whole batch(es) of B={B} L={a['input_ids'].shape[1]} through the batched torch fp32 "
                      f"restatement of the reference graph (24 layers + classifier, every row at full length), "
                      f"{el:.1f} s")
    if gpu_logits is not None:  # the fp16 GPU chain against the fp32 CPU graph
        out["max_abs_logit_diff_vs_gpu"] = round(float(np.max(np.abs(logits.numpy() - gpu_logits))), 5)
    return out


def single_layer_us(model, iters=200):
    """One encoder layer at B=1, L=32 (hidden N(0,1), all-ones mask) through
    gd_classifier_layer_forward, HIP events around `iters` back-to-back calls
    on the launch stream.  Its bound: the layer's 25.2 MB of weights read
    once at 8 TB/s."""
    import torch
    from gliner_decide.synthetic import layer_inputs
    d = layer_inputs(seed=1)
    h = torch.from_numpy(d["hidden"]).cuda()
    mask = torch.from_numpy(d["mask"]).cuda()
    for _ in range(10):
        model.layer_forward(0, h, mask)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        model.layer_forward(0, h, mask)
    end.record()
    end.synchronize()
    us = start.elapsed_time(end) * 1000.0 / iters
    C, F = 1024, 4096
    wbytes = (4 * C * C + 2 * C * F) * 2 + (6 * C + F + 4 * C) * 2
    return dict(us=round(us, 2), weight_bytes=wbytes, bound_us=round(wbytes / HBM_PEAK_GBS / 1e3, 2),
                frac_of_bound=round(wbytes / HBM_PEAK_GBS / 1e3 / us, 4), iters=iters,
                sample="gd_classifier_layer_forward, B=1 L=32, layer 0 of the 24-layer model")


def long_context_rate(model, steps=5, warmup=2):
    """Rows/s at B=64, L=512 (every row full, 3 heads of 20/20/8 labels),
    packed classify with inputs in HBM."""
    import torch
    from gliner_decide import DecisionInput
    from gliner_decide.decode import row_extents
    from gliner_decide.synthetic import long_context_batch
    batch = long_context_batch(seed=6)
    a = batch.arrays()
    ids, mask, mk, mm = DecisionInput(**a).to_device()
    B, L = ids.shape
    model.reserve(B, L, mk.shape[1], mk.shape[2])
    out = torch.empty((B, mk.shape[1], mk.shape[2]), dtype=torch.float16, device=ids.device)
    total = int(row_extents(a["attention_mask"], a["marker_indices"], a["marker_mask"]).sum())
    for _ in range(warmup):
        model.classify_device(ids, mask, mk, mm, out, total_tokens=total)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.classify_device(ids, mask, mk, mm, out, total_tokens=total)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    assert torch.isfinite(out.float()).all()
    return dict(value=round(B * steps / el, 1), unit="rows/s", ms_per_step=round(el * 1000 / steps, 3), steps=steps,
                sample="B=64 L=512 full rows, 3 heads (20/20/8 labels), packed classify")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this path is data-parallel "
              "over independent rows and runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from gliner_decide import DecisionInput, GLiNERDecideClassifier
    from gliner_decide.config import DeBERTaV2Configuration
    from gliner_decide.decode import row_extents
    from gliner_decide.synthetic import classification_batch, long_context_batch, synthetic_weights

    torch.cuda.set_device(0)
    cfg = DeBERTaV2Configuration(vocab_size=128100)
    if not args.profile_kernel and not args.serving:
        # the roofline kernel first: the launch sequence of --profile-kernel in
        # the same process state (nothing has run on the GPU yet)
        roof_k = measure_kernels(cfg, args.kernel_iters, only=ROOFLINE_KERNEL)[ROOFLINE_KERNEL]
        log(f"{ROOFLINE_KERNEL}: {roof_k['us']:.2f} us per launch over {args.kernel_iters} launches")
    if args.profile_kernel:
        kernels = measure_kernels(cfg, args.kernel_iters, only=args.profile_kernel)
        nb = calibration_copy()
        for k, v in kernels.items():
            log(f"{k}: {v['us']:.2f} us per launch over {args.kernel_iters} launches; calibration copy {nb} B")
        return
    if args.profile_layer:
        cfg1 = DeBERTaV2Configuration(vocab_size=128100, num_hidden_layers=1)
        layer = single_layer_us(GLiNERDecideClassifier(synthetic_weights(cfg1, seed=4), cfg1))
        log(f"single layer B=1 L=32: {layer['us']:.2f} us per call over {layer['iters']} calls")
        return
    t = time.perf_counter()
    weights = synthetic_weights(cfg, seed=4)
    log(f"weights generated in {time.perf_counter() - t:.1f} s")
    if args.serving:
        srv = serving_rate(weights, cfg)
        log(f"serving: {srv}")
        print(json.dumps({"metric": "rows/s, JSONL serving (text to decisions), 24L encoder + cls head",
                          "value": srv["value"], "unit": "rows/s", "n_gpus": 1, "higher_is_better": True,
                          "dtype": "f16", "data": "synthetic (seeded texts and task schemas; random-init weights)",
                          "config": {"workload": "JSONL runner over the bucket-mix text workload", "batch": 32},
                          "serving": srv}), flush=True)
        return
    model = GLiNERDecideClassifier(weights, cfg, use_compiled_graph=args.compiled)
    log(f"model on device: {model.device_bytes / 2**20:.0f} MiB")
    if args.bucket_mix:
        mix = bucket_mix_rate(model)
        log(f"bucket mix: {mix}")
        print(json.dumps({"metric": "rows/s, bucket mix (B=32 batches over L32..L512), 24L encoder + cls head",
                          "value": mix["value"], "unit": "rows/s", "n_gpus": 1, "higher_is_better": True,
                          "dtype": "f16", "data": "synthetic (seeded ids/lengths; random-init weights)",
                          "config": {"workload": "bucket mix: 4096 rows, lengths exp(U(ln 8, ln 512)), 1-2 tasks x "
                                                 "2-10 labels, packed rows", "batch": 32,
                                     "compiled_graph": args.compiled},
                          "bucket_mix": mix}), flush=True)
        return
    if args.workload == "classify":
        batch = classification_batch(seed=4)
        wl = dict(workload="24L DeBERTa-v3-large encoder + GLiNER classifier head, B=32 L=256 "
                           "(lengths U[40,256], 1 task x 5 labels)", global_batch=32, seq_len=256)
    else:
        batch = long_context_batch(seed=6)
        wl = dict(workload="24L encoder + classifier, B=64 L=512 full rows, 3 heads (20/20/8 labels)",
                  global_batch=64, seq_len=512)
    host = batch.arrays()
    ids, mask, markers, mmask = DecisionInput(**host).to_device()
    B, L = ids.shape
    _, Hh, O_ = markers.shape
    model.reserve(B, L, Hh, O_)
    logits = torch.empty((B, Hh, O_), dtype=torch.float16, device=ids.device)
    # The step ends with the logits in host memory (main.swift:247-279 reads
    # them back): an asynchronous copy into pinned memory on the forward's
    # stream, so the next step's forward queues behind it without a host wait.
    logits_host = torch.empty((B, Hh, O_), dtype=torch.float16, pin_memory=True)

    def step():
        # the packed forward's token count comes from the host copy of the
        # batch (what a tokenizer knows), every step
        total = int(row_extents(host["attention_mask"], host["marker_indices"], host["marker_mask"]).sum())
        model.classify_device(ids, mask, markers, mmask, logits, total_tokens=total)
        logits_host.copy_(logits, non_blocking=True)

    def timed(fn, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    for _ in range(args.warmup):
        step()
    elapsed = timed(step, args.steps)
    ms = elapsed * 1000 / args.steps
    rows_s = B * args.steps / elapsed
    assert torch.isfinite(logits.float()).all()
    assert torch.equal(logits_host, logits.cpu())
    packed_logits = logits.clone()  # the headline forward's output
    log(f"e2e: {ms:.3f} ms/step, {rows_s:.1f} rows/s (packed rows, logits read back to pinned host memory)")
    padded_logits = torch.empty_like(logits)
    padded = lambda: model.classify_device(ids, mask, markers, mmask, padded_logits)  # noqa: E731
    for _ in range(args.warmup):
        padded()
    padded_s = timed(padded, args.steps)
    log(f"e2e padded: {padded_s * 1000 / args.steps:.3f} ms/step, {B * args.steps / padded_s:.1f} rows/s")
    # The reference's amount of work: every position of every layer (GD_FULL_ROWS);
    # the logits must equal the row-extent / marker-row forward's bit for bit.
    full = GLiNERDecideClassifier(weights, cfg, use_compiled_graph=args.compiled, full_rows=True)
    full.reserve(B, L, Hh, O_)
    full_logits = torch.empty_like(logits)
    full_step = lambda: full.classify_device(ids, mask, markers, mmask, full_logits)  # noqa: E731
    for _ in range(args.warmup):
        full_step()
    full_s = timed(full_step, args.steps)
    assert torch.equal(full_logits, packed_logits), "full-row logits differ from the packed (headline) forward's"
    assert torch.equal(full_logits, padded_logits), "full-row logits differ from the padded forward's"
    log(f"e2e full rows: {full_s * 1000 / args.steps:.3f} ms/step, {B * args.steps / full_s:.1f} rows/s")
    full.close()
    del full
    # The reference's batch loop (main.swift:259-276): host arrays in, each
    # batch's forward waited for and its logits read back before the next.
    # PCIe-inclusive and synchronous; never `value`.
    host_inp = DecisionInput(**host)
    host_step = lambda: model.classify(host_inp).logits.cpu()  # noqa: E731
    for _ in range(args.warmup):
        host_step()
    host_s = timed(host_step, args.steps)
    assert torch.equal(model.classify(host_inp).logits, packed_logits), "host-array logits differ"
    log(f"e2e host arrays, synchronous: {host_s * 1000 / args.steps:.3f} ms/step, {B * args.steps / host_s:.1f} rows/s")

    kernels = measure_kernels(cfg, args.kernel_iters)
    for k, v in kernels.items():
        extra = f"{v['gbs']:.0f} GB/s" if "gbs" in v and v["bound"] == "hbm" else f"{v.get('tflops', 0):.0f} TFLOP/s"
        log(f"  {k:20s} {v['us']:9.2f} us  {extra}")
    roof = roofline_of(ROOFLINE_KERNEL, roof_k, args.kernel_iters)
    layer1 = single_layer_us(model)
    log(f"single layer B=1 L=32: {layer1}")
    longctx = long_context_rate(model) if args.workload == "classify" else None
    log(f"long context B=64 L=512: {longctx}")

    # after the kernel table: seconds of sustained load change the clocks the
    # short kernels above would be timed at
    mix = None
    if args.workload == "classify" and not args.no_bucket_mix:
        mix = bucket_mix_rate(model)
        log(f"bucket mix: {mix}")

    cpu = None
    if not args.no_cpu_baseline and args.workload == "classify":
        cpu = cpu_baseline(weights, cfg, batch, args.cpu_seconds, packed_logits.float().cpu().numpy())
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": "rows/s, 24L encoder+cls head B=32 L=256; fused LN/rel-bias GB/s vs HBM peak",
        "value": round(rows_s, 2),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded ids/lengths; random-init N(0,0.02) fp16 weights of DeBERTa-v3-large + GLiNER head)",
        "config": dict(wl, parallelism="single GPU", compiled_graph=args.compiled, rows="packed",
                       step="forward + classifier + logits D2H into pinned host memory"),
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernels": {k: dict({kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()},
                            traffic=profiled_traffic(k)[0])
                    for k, v in kernels.items()},
        "fused_ln_gbs": round(kernels["residual_layernorm"]["gbs"], 1),
        "fused_ln_frac_hbm": round(kernels["residual_layernorm"]["gbs"] / HBM_PEAK_GBS, 4),
        "stream_ceiling_gbs": round(kernels["stream_ceiling"]["gbs"], 1),
        "fused_ln_frac_of_stream_ceiling": round(kernels["residual_layernorm"]["gbs"] / kernels["stream_ceiling"]["gbs"],
                                                 4),
        "relbias_softmax_gbs": round(kernels["relbias_softmax"]["gbs"], 1),
        "relbias_softmax_frac_hbm": round(kernels["relbias_softmax"]["gbs"] / HBM_PEAK_GBS, 4),
        "bucket_mix_rows_s": mix,
        "padded_rows_s": round(B * args.steps / padded_s, 2),
        "full_rows_s": round(B * args.steps / full_s, 2),
        "host_sync_rows_s": round(B * args.steps / host_s, 2),
        "relative_bias_gbs": round(kernels["relative_bias"]["gbs"], 1),
        "relative_bias_frac_hbm": round(kernels["relative_bias"]["gbs"] / HBM_PEAK_GBS, 4),
        "single_layer_b1_l32": layer1,
        "long_context_b64_l512_rows_s": longctx,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
