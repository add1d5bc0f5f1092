"""Benchmark of the HIP paged-attention path on one MI355X.

Headline workload (one "step"): paged GQA decode, fp16, batch 32, every
context 2048 tokens, Hq=16 / Hkv=8 / D=128, block size 256, 28 layers run
back-to-back, each layer with its own KV pool (263 pages), own queries and
own random non-contiguous block table (Qwen3-0.6B decode-step shapes).
Inputs are synthetic N(0,1), resident in HBM before timing starts.

Timing: a HIP graph holds the 28 layer calls; W warm-up replays, then K
timed replays bracketed by synchronisation, HIP events on the launch stream.
value = algorithmic HBM bytes of a step / step time (TB/s); algorithmic
bytes count every KV row of a layer once (4096 B per token per layer) plus
q, out, tables and lengths: 268,699,904 B per layer.

Also reported (field "extra"): the other workloads of the same path --
B=1/ctx128, B=8/ctx512 with the KV scatter, ragged B=64 with a shared
prefix, and chunked prefill 8x128 on MFMA.

The CPU leg (field "cpu_baseline", off with --no-cpu-baseline) is the only
part that touches the oracle: it times the reference's torch path (restated
in the oracle) on this host on bounded samples -- one headline decode
layer, and the chunked-prefill workload's KV scatter and prefill attention
-- and computes the reference outputs that every GPU
result above is compared with (the error fields are null without it).

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
from pathlib import Path
import platform
import statistics
import subprocess
import sys
import time

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "myvllm-mini-engine_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "paged-decode µs/call + HBM TB/s (% peak), B=32 ctx2048 Hq16/Hkv8/D128"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
LAYERS = 28
BATCH, CONTEXT, BLOCK = 32, 2048, 256
HQ, HKV, D = 16, 8, 128
BASE_SEED = 20261026
DECODE_NAMES = ("query", "key_cache", "value_cache", "block_tables", "context_lens")
REFERENCE_US_PER_CALL = 362.44  # RTX 5080, block 256 fp16, decode_numerical_round_20261102.json:1693


def layer_bytes(batch=BATCH, context=CONTEXT, width=CONTEXT // BLOCK):
    kv = batch * context * HKV * D * 2 * 2
    return kv + 2 * batch * HQ * D * 2 + batch * width * 8 + batch * 8


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def graph_time_ms(fn, torch, *, calls_per_graph, replays, warmup):
    """Capture `fn` (which issues calls_per_graph calls) once, time replays."""
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / replays, graph


def eager_wall_ms(fn, torch, repeats=5):
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(repeats):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / repeats


def max_abs(actual, expected):
    return (actual.float().cpu() - expected.float().cpu()).abs().max().item()


# ---------------------------------------------------------------------------
# Headline: 28-layer decode step.
# ---------------------------------------------------------------------------

def headline(args, torch, paged_attention, workloads):
    dev = torch.device("cuda:0")
    layers = []
    for layer in range(LAYERS):
        case = workloads.decode_b32_layer(dev, seed=BASE_SEED + 2 + 1000 * layer)
        case["out"] = torch.empty_like(case["query"])
        layers.append(case)
    torch.cuda.synchronize()
    log(f"headline inputs resident: {LAYERS} layers x 2 x {layers[0]['key_cache'].numel() * 2 / 2**20:.1f} MiB")

    def step():
        for c in layers:
            paged_attention(c["query"], c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"],
                            BLOCK, backend="hip", validate=False, partition_tokens=args.partition,
                            out=c["out"])

    ms, graph = graph_time_ms(step, torch, calls_per_graph=LAYERS, replays=args.steps, warmup=args.warmup)
    eager_ms = eager_wall_ms(step, torch, repeats=3)
    return layers, ms, eager_ms


def headline_parity(layers, cpu):
    """Layer 0 and layer 27 against the fp32 reference (fp16 gate 2e-3)."""
    worst = 0.0
    for idx in (0, LAYERS - 1):
        c = layers[idx]
        tensors = {"query": c["query"].cpu(), "key_cache": c["key_cache"].cpu(), "value_cache": c["value_cache"].cpu(),
                   "block_tables": c["block_tables"].cpu(), "context_lens": c["context_lens"].cpu()}
        worst = max(worst, max_abs(c["out"], cpu.decode(tensors, BLOCK)))
    return {"layers_checked": [0, LAYERS - 1], "max_abs_error": worst, "gate": 2e-3, "passed": worst <= 2e-3}


def decode_step_with_scatter(args, torch, layers, write_kv_cache_batch, paged_attention, cpu):
    """The decode step as the engine runs it per layer (native_qwen3.py:179-197):
    write the batch's new K/V row at position len-1 of every sequence
    (write_kv_cache_batch), then paged attention over the updated context --
    28 layers in one captured graph (the "--cuda-graph" decode step with the
    hip backend).  Reuses the headline layers; changes their last KV row."""
    gen = torch.Generator(device="cuda").manual_seed(BASE_SEED + 77)
    for c in layers:
        c["new_key"] = torch.randn((BATCH, HKV, D), generator=gen, device="cuda").half()
        c["new_value"] = torch.randn((BATCH, HKV, D), generator=gen, device="cuda").half()
        c["offsets"] = (c["context_lens"] - 1).contiguous()

    def step():
        for c in layers:
            write_kv_cache_batch(c["key_cache"], c["value_cache"], c["block_tables"], c["offsets"], c["new_key"],
                                 c["new_value"], BLOCK, backend="hip", validate=False)
            paged_attention(c["query"], c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"],
                            BLOCK, backend="hip", validate=False, out=c["out"])

    ms, _ = graph_time_ms(step, torch, calls_per_graph=2 * LAYERS, replays=args.steps, warmup=args.warmup)
    c = layers[0]
    tables, offsets = c["block_tables"].cpu(), c["offsets"].cpu()
    pages = tables[torch.arange(BATCH), offsets // BLOCK]
    rows_k = c["key_cache"].cpu()[pages, offsets % BLOCK]
    rows_v = c["value_cache"].cpu()[pages, offsets % BLOCK]
    scatter_ok = torch.equal(rows_k, c["new_key"].cpu()) and torch.equal(rows_v, c["new_value"].cpu())
    err = None
    if cpu is not None:
        tensors = {"query": c["query"].cpu(), "key_cache": c["key_cache"].cpu(),
                   "value_cache": c["value_cache"].cpu(), "block_tables": tables,
                   "context_lens": c["context_lens"].cpu()}
        err = max_abs(c["out"], cpu.decode(tensors, BLOCK))
    # The same step with the write fused into the attention launch
    # (paged_attention_decode_write): results equal the two launches bit for bit.
    from mini_engine_hip.kernels.paged import paged_attention_decode_write
    want = [c["out"].clone() for c in layers]
    for c in layers:
        c["out"].zero_()

    def fused_step():
        for c in layers:
            paged_attention_decode_write(c["query"], c["key_cache"], c["value_cache"], c["block_tables"],
                                         c["context_lens"], BLOCK, c["new_key"], c["new_value"], validate=False,
                                         out=c["out"])

    ms_fused, _ = graph_time_ms(fused_step, torch, calls_per_graph=LAYERS, replays=args.steps, warmup=args.warmup)
    fused_equal = all(torch.equal(c["out"], w) for c, w in zip(layers, want))
    step_bytes = LAYERS * (layer_bytes() + 2 * BATCH * HKV * D * 2 * 2 + BATCH * 8)
    return {"us_per_step": ms * 1e3, "us_per_layer": ms * 1e3 / LAYERS,
            "TBps": step_bytes / (ms * 1e-3) / 1e12, "launches_per_step": 2 * LAYERS,
            "scatter_bit_exact": scatter_ok, "max_abs_error_layer0": err, "gate": 2e-3,
            "fused_write_us_per_layer": ms_fused * 1e3 / LAYERS, "fused_write_launches_per_step": LAYERS,
            "fused_write_equals_two_launches": fused_equal,
            "passed": scatter_ok and fused_equal and (err is None or err <= 2e-3)}


def decode_attention_block_step(args, torch, layers, paged_attention, cpu):
    """The attention block of the decode step for all 28 headline layers in one captured graph:
    per layer the fused q/k RMSNorm + RoPE + KV page write of the new token (replacing q_norm,
    k_norm, apply_rope and write_kv_cache_batch, native_qwen3.py:179-191), paged attention over
    the updated context, and the o_proj projection of the batch (mvme_linear_rows, HipLinear's
    decode-batch kernel; native_qwen3.py:197).
    Inputs are synthetic QKV projections of the batch; reuses the headline layers' caches."""
    from mini_engine_hip.kernels.rope import qk_norm_rope_write_kv
    from mini_engine_hip.kernels.linear import linear_rows

    hidden = 2048
    gen = torch.Generator(device="cuda").manual_seed(BASE_SEED + 99)
    for c in layers:
        c["qkv"] = torch.randn((BATCH, (HQ + 2 * HKV) * D), generator=gen, device="cuda").half()
        c["wq"] = (torch.rand((D,), generator=gen, device="cuda") + 0.5).half()
        c["wk"] = (torch.rand((D,), generator=gen, device="cuda") + 0.5).half()
        angles = torch.randn((BATCH, D // 2), generator=gen, device="cuda")
        c["cos"], c["sin"] = angles.cos().half(), angles.sin().half()
        c["w_o"] = (torch.randn((hidden, HQ * D), generator=gen, device="cuda") * 0.02).half()  # [out, in]
        c["positions"] = (c["context_lens"] - 1).contiguous()
        c["q_rot"] = torch.empty((BATCH, HQ, D), dtype=torch.float16, device="cuda")
        c["hidden"] = torch.empty((BATCH, hidden), dtype=torch.float16, device="cuda")

    def split(c):
        q = c["qkv"][:, :HQ * D].view(BATCH, HQ, D)
        k = c["qkv"][:, HQ * D:(HQ + HKV) * D].view(BATCH, HKV, D)
        v = c["qkv"][:, (HQ + HKV) * D:].view(BATCH, HKV, D)
        return q, k, v

    def step():
        for c in layers:
            q, k, v = split(c)
            qk_norm_rope_write_kv(q, k, v, c["wq"], c["wk"], c["cos"], c["sin"], c["key_cache"], c["value_cache"],
                                  block_tables=c["block_tables"], positions=c["positions"], validate=False,
                                  out=c["q_rot"])
            paged_attention(c["q_rot"], c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"],
                            BLOCK, backend="hip", validate=False, out=c["out"])
            linear_rows(c["out"].view(BATCH, HQ * D), c["w_o"], out=c["hidden"])

    ms, _ = graph_time_ms(step, torch, calls_per_graph=3 * LAYERS, replays=args.steps, warmup=args.warmup)
    # Layer 0 against the reference: the rotated q, the written K/V rows, attention, o_proj.
    c = layers[0]
    v_exact = rope_err = attn_err = o_err = passed = None
    if cpu is not None:
        q, k, v = (t.cpu() for t in split(c))
        tables, positions = c["block_tables"].cpu(), c["positions"].cpu()
        kc, vc = c["key_cache"].cpu(), c["value_cache"].cpu()
        kc_o, vc_o = kc.clone(), vc.clone()
        q_ref = cpu.norm_rope_write_kv(q, k, v, c["wq"].cpu(), c["wk"].cpu(), c["cos"].cpu(), c["sin"].cpu(),
                                       kc_o, vc_o, block_tables=tables, positions=positions)
        rope_err = max(max_abs(c["q_rot"], q_ref), max_abs(kc, kc_o))
        v_exact = torch.equal(vc, vc_o)
        tensors = {"query": c["q_rot"].cpu(), "key_cache": kc, "value_cache": vc, "block_tables": tables,
                   "context_lens": c["context_lens"].cpu()}
        attn_err = max_abs(c["out"], cpu.decode(tensors, BLOCK))
        o_err = max_abs(c["hidden"], c["out"].float().cpu().view(BATCH, -1) @ c["w_o"].float().cpu().t())
        passed = v_exact and rope_err <= 4e-3 and attn_err <= 2e-3 and o_err <= 2e-2
    # The same block with norm/RoPE and the KV write fused into the attention
    # launch (paged_attention_decode_write), then o_proj: two launches per layer.
    from mini_engine_hip.kernels.paged import paged_attention_decode_write
    want = [(c["q_rot"].clone(), c["out"].clone(), c["hidden"].clone()) for c in layers]
    for c in layers:
        c["q_rot"].zero_()
        c["out"].zero_()
        c["hidden"].zero_()

    def fused_step():
        for c in layers:
            q, k, v = split(c)
            paged_attention_decode_write(q, c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"],
                                         BLOCK, k, v, q_weight=c["wq"], k_weight=c["wk"], cos=c["cos"],
                                         sin=c["sin"], q_out=c["q_rot"], validate=False, out=c["out"])
            linear_rows(c["out"].view(BATCH, HQ * D), c["w_o"], out=c["hidden"])

    ms_fused, _ = graph_time_ms(fused_step, torch, calls_per_graph=2 * LAYERS, replays=args.steps,
                                warmup=args.warmup)
    fused_equal = all(torch.equal(c["q_rot"], w[0]) and torch.equal(c["out"], w[1]) and torch.equal(c["hidden"], w[2])
                      for c, w in zip(layers, want))
    if passed is not None:
        passed = passed and fused_equal
    for c in layers:
        for key in ("qkv", "wq", "wk", "cos", "sin", "w_o", "positions", "q_rot", "hidden"):
            del c[key]
    return {"us_per_step": ms * 1e3, "us_per_layer": ms * 1e3 / LAYERS, "launches_per_step": 3 * LAYERS,
            "v_rows_bit_exact": v_exact, "max_abs_error_rope_layer0": rope_err,
            "max_abs_error_attention_layer0": attn_err, "max_abs_error_o_proj_layer0": o_err,
            "fused_prologue_us_per_layer": ms_fused * 1e3 / LAYERS, "fused_prologue_launches_per_step": 2 * LAYERS,
            "fused_prologue_equals_three_launches": fused_equal, "passed": passed}


def _median_seconds(fn, budget_s, min_runs=5, max_runs=20):
    """Median wall time of fn() after one warm-up: at least min_runs runs, more
    while inside the budget (never past 3x the budget)."""
    fn()
    samples = []
    t_start = time.perf_counter()
    while len(samples) < min_runs or (time.perf_counter() - t_start < budget_s and len(samples) < max_runs):
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    return statistics.median(samples), len(samples)


class CpuLeg:
    """The CPU leg: the reference's torch path restated in the oracle, on the
    host cores.  It is the only user of the oracle in this file -- as the
    timed CPU baseline and to compute the reference outputs
    the GPU results are compared with."""

    def __init__(self, torch):
        from oracle import paged_oracle

        self.torch = torch
        self.oracle = paged_oracle

    # Reference outputs (the oracle).
    def decode(self, tensors, block_size):
        return self.oracle.fp32_oracle(tensors, block_size)

    def prefill(self, *args, **kwargs):
        return self.oracle.paged_prefill_attention(*args, **kwargs)

    def dense_prefill(self, *args, **kwargs):
        return self.oracle.prefill_attention(*args, **kwargs)

    def norm_rope_write_kv(self, *args, **kwargs):
        return self.oracle.qk_norm_rope_write_kv(*args, **kwargs)

    def greedy(self, logits):
        return self.oracle.greedy_argmax(logits)

    # Timed baselines.
    def cpu_model(self):
        model = platform.processor() or ""
        try:
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
            for line in out.splitlines():
                if line.startswith("Model name:"):
                    model = line.split(":", 1)[1].strip()
        except Exception:
            pass
        return model

    def baseline(self, workloads, budget_s):
        """Headline fields (one decode layer), plus the chunked-prefill workload's
        scatter and prefill attention under "other_workloads"."""
        torch = self.torch
        threads = torch.get_num_threads()
        c = workloads.decode_b32_layer(torch.device("cuda:0"), seed=BASE_SEED + 2)
        tensors = [c["query"].cpu(), c["key_cache"].cpu(), c["value_cache"].cpu(), c["block_tables"].cpu(),
                   c["context_lens"].cpu()]
        del c
        sec, runs = _median_seconds(lambda: self.oracle.paged_attention(*tensors, BLOCK), budget_s)
        del tensors
        cpu_model = self.cpu_model()
        result = {"value": layer_bytes() / sec / 1e12, "unit": "TB/s", "cores": threads, "kind": "port",
                  "us_per_call": sec * 1e6,
                  "sample": (f"one layer of the headline step (B=32, ctx 2048, fp16, block 256) through the "
                             f"reference's torch decode path (fallback.py:27-64, restated in oracle/paged_oracle.py); "
                             f"median of {runs} runs after 1 warm-up; torch threads={threads}, "
                             f"os.cpu_count()={os.cpu_count()}, cpu={cpu_model}")}
        # Chunked prefill 8 x 128 (bf16, block 256): the reference's torch scatter
        # (index_copy_, data.py:120-125) and torch prefill (prefill.py:114-131).
        pc = workloads.chunked_prefill_case(device=torch.device("cuda:0"))
        cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in pc.items()}
        del pc
        kc, vc = cpu["key_cache"].clone(), cpu["value_cache"].clone()
        scatter = lambda: self.oracle.write_kv_cache_slots(kc, vc, cpu["slot_mapping"], cpu["new_key"],  # noqa: E731
                                                           cpu["new_value"])
        s_sec, s_runs = _median_seconds(scatter, budget_s / 4)
        names = ("q", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
        q, cu, st, tb, ln = (cpu[n] for n in names)
        prefill = lambda: self.oracle.paged_prefill_attention(q, kc, vc, cu, st, tb, ln, 256)  # noqa: E731
        p_sec, p_runs = _median_seconds(prefill, budget_s / 2)
        flops = workloads.prefill_flops(cpu["priors"])
        moved = 2 * 1024 * HKV * D * 2 * 2 + 1024 * 8
        result["other_workloads"] = {
            "kv_scatter_1024_tokens_bf16": {
                "us_per_call": s_sec * 1e6, "GBps": moved / s_sec / 1e9,
                "sample": f"the 1024 new K/V rows of the chunked-prefill workload, median of {s_runs} runs"},
            "chunked_prefill_8x128_bf16": {
                "us_per_call": p_sec * 1e6, "TFLOPs": flops / p_sec / 1e12,
                "sample": f"8 sequences x 128 new tokens, priors {cpu['priors']}, median of {p_runs} runs"}}
        return result


# ---------------------------------------------------------------------------
# Other workloads of the path (reported under "extra").
# ---------------------------------------------------------------------------

EXTRA_NAMES = ("decode_b1", "decode_b8", "ragged_b64", "decode_shards", "prefill", "prefill_shapes", "dense_prefill",
               "kv_scatter", "norm_rope", "after_attention")


def extra_workloads(torch, paged_attention, write_kv_cache_slots, paged_prefill_attention, workloads, cpu,
                    names=EXTRA_NAMES):
    dev = torch.device("cuda:0")
    extra = {}
    if "decode_b1" in names:
        _extra_b1(torch, paged_attention, workloads, cpu, dev, extra)
    if "decode_b8" in names:
        _extra_b8(torch, paged_attention, write_kv_cache_slots, workloads, cpu, dev, extra)
    if "ragged_b64" in names:
        _extra_ragged(torch, paged_attention, workloads, cpu, dev, extra)
    if "decode_shards" in names:
        _extra_shards(torch, paged_attention, cpu, dev, extra)
    if "prefill" in names:
        _extra_prefill(torch, write_kv_cache_slots, paged_prefill_attention, workloads, cpu, dev, extra)
        _extra_prefill_cold(torch, write_kv_cache_slots, paged_prefill_attention, workloads, cpu, dev, extra)
    if "prefill_shapes" in names:
        _extra_prefill_shapes(torch, write_kv_cache_slots, paged_prefill_attention, workloads, dev, extra)
    if "dense_prefill" in names:
        _extra_dense_prefill(torch, workloads, cpu, dev, extra)
    if "kv_scatter" in names:
        _extra_kv_scatter(torch, write_kv_cache_slots, workloads, cpu, dev, extra)
    if "norm_rope" in names:
        _extra_norm_rope(torch, cpu, dev, extra)
    if "after_attention" in names:
        _extra_after_attention(torch, cpu, dev, extra)
    return extra


def _extra_b1(torch, paged_attention, workloads, cpu, dev, extra):
    # B=1 / ctx 128, fp16, block 256.
    c = workloads.decode_b1(dev)
    out = torch.empty_like(c["query"])
    fn = lambda: paged_attention(c["query"], c["key_cache"], c["value_cache"], c["block_tables"],  # noqa: E731
                                 c["context_lens"], 256, backend="hip", validate=False, out=out)

    def many(n=50):
        def run():
            for _ in range(n):
                fn()
        return run
    ms, _ = graph_time_ms(many(), torch, calls_per_graph=50, replays=20, warmup=3)
    err = None if cpu is None else max_abs(out, cpu.decode({k: c[k].cpu() for k in DECODE_NAMES}, 256))
    bytes_b1 = 1 * 128 * 4096 + 2 * 16 * 128 * 2 + 8 + 8
    extra["decode_b1_ctx128_fp16"] = {"us_per_call": ms / 50 * 1e3, "GBps": bytes_b1 / (ms / 50 * 1e-3) / 1e9,
                                      "max_abs_error": err, "reference_rtx5080_us": 18.945}


def _extra_b8(torch, paged_attention, write_kv_cache_slots, workloads, cpu, dev, extra):
    # B=8 / ctx 512, bf16, block 16, + scatter of the new token.
    c = workloads.decode_b8_with_scatter(dev)
    out = torch.empty_like(c["query"])

    def scatter_decode():
        write_kv_cache_slots(c["key_cache"], c["value_cache"], c["slot_mapping"], c["new_key"], c["new_value"],
                             backend="hip", validate=False)
        paged_attention(c["query"], c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"], 16,
                        backend="hip", validate=False, out=out)

    def many2(n=50):
        def run():
            for _ in range(n):
                scatter_decode()
        return run
    ms, _ = graph_time_ms(many2(), torch, calls_per_graph=50, replays=20, warmup=3)
    kc, vc = c["key_cache"].cpu(), c["value_cache"].cpu()
    slots_ok = torch.equal(kc.view(-1, 8, 128)[c["slot_mapping"].cpu()], c["new_key"].cpu())
    err = None
    if cpu is not None:
        err = max_abs(out, cpu.decode({"query": c["query"].cpu(), "key_cache": kc, "value_cache": vc,
                                       "block_tables": c["block_tables"].cpu(),
                                       "context_lens": c["context_lens"].cpu()}, 16))
    # The same step with the write inside the attention launch (the new token
    # sits at position len - 1 = 511 of every sequence).
    from mini_engine_hip.kernels.paged import paged_attention_decode_write
    out_fused = torch.empty_like(out)

    def fused(n=50):
        def run():
            for _ in range(n):
                paged_attention_decode_write(c["query"], c["key_cache"], c["value_cache"], c["block_tables"],
                                             c["context_lens"], 16, c["new_key"], c["new_value"], validate=False,
                                             out=out_fused)
        return run
    ms_fused, _ = graph_time_ms(fused(), torch, calls_per_graph=50, replays=20, warmup=3)
    bytes_b8 = 8 * 512 * 4096 + 2 * 8 * 16 * 128 * 2 + 8 * 32 * 8 + 8 * 8
    extra["decode_b8_ctx512_bf16_with_scatter"] = {
        "us_per_call": ms / 50 * 1e3, "GBps_decode_bytes": bytes_b8 / (ms / 50 * 1e-3) / 1e9,
        "scatter_bit_exact": bool(slots_ok), "max_abs_error": err, "reference_rtx5080_us": 40.340,
        "fused_write_us_per_call": ms_fused / 50 * 1e3,
        "fused_write_equals_two_launches": bool(torch.equal(out_fused, out))}


def _extra_ragged(torch, paged_attention, workloads, cpu, dev, extra):
    # Ragged B=64, ctx U[1,4096], bf16, block 16, shared 1024-token prefix.
    c = workloads.ragged_shared_prefix_case(device=dev)
    out = torch.empty_like(c["query"])
    fn4 = lambda: paged_attention(c["query"], c["key_cache"], c["value_cache"], c["block_tables"],  # noqa: E731
                                  c["context_lens"], 16, backend="hip", validate=False, out=out)

    def many4(n=10):
        def run():
            for _ in range(n):
                fn4()
        return run
    ms, _ = graph_time_ms(many4(), torch, calls_per_graph=10, replays=10, warmup=2)
    per_call = ms / 10 * 1e-3
    unique = c["unique_rows"] * 4096 + 2 * 64 * 16 * 128 * 2 + 64 * 256 * 8 + 64 * 8
    logical = c["logical_rows"] * 4096 + 2 * 64 * 16 * 128 * 2 + 64 * 256 * 8 + 64 * 8
    err = None if cpu is None else max_abs(out, cpu.decode({k: c[k].cpu() for k in DECODE_NAMES}, 16))
    extra["ragged_b64_shared_prefix_bf16"] = {
        "us_per_call": per_call * 1e6, "GBps_unique": unique / per_call / 1e9,
        "frac_of_hbm_peak_unique": unique / per_call / 1e9 / HBM_PEAK_GBS,
        "GBps_logical": logical / per_call / 1e9, "unique_rows": c["unique_rows"], "logical_rows": c["logical_rows"],
        "max_abs_error": err}
    del c, out
    # Ragged B=32, ctx U[1,4096], fp16, block 256: one unit per CU, each with
    # 2 MiB of K+V capacity, so the plan takes the balanced walk.
    r = workloads.ragged_decode_case(device=dev)
    rout = torch.empty_like(r["query"])
    fnr = lambda: paged_attention(r["query"], r["key_cache"], r["value_cache"], r["block_tables"],  # noqa: E731
                                  r["context_lens"], 256, backend="hip", validate=False, out=rout)

    def manyr(n=10):
        def run():
            for _ in range(n):
                fnr()
        return run
    ms, _ = graph_time_ms(manyr(), torch, calls_per_graph=10, replays=10, warmup=2)
    per_call = ms / 10 * 1e-3
    rows = int(r["context_lens"].sum())
    nbytes = rows * 4096 + 2 * 32 * 16 * 128 * 2 + 32 * 16 * 8 + 32 * 8
    err = None if cpu is None else max_abs(rout, cpu.decode({k: r[k].cpu() for k in DECODE_NAMES}, 256))
    extra["ragged_b32_ctx4096_fp16_balanced_walk"] = {
        "us_per_call": per_call * 1e6, "GBps": nbytes / per_call / 1e9,
        "frac_of_hbm_peak": nbytes / per_call / 1e9 / HBM_PEAK_GBS, "rows": rows, "algorithmic_bytes": nbytes,
        "max_abs_error": err}
    del r, rout
    # Ragged B=16, ctx U[1,8192], bf16, block 16: 128 long units on 256 CUs.
    # The plan takes the balanced walk; split-K with the partitions sized
    # from the capacity (2048 tokens: two work-groups per CU) is timed beside it.
    w = workloads.ragged_decode_case(device=dev, batch=16, max_len=8192, block_size=16, dtype=torch.bfloat16,
                                     seed=BASE_SEED + 6)
    wout = torch.empty_like(w["query"])
    ws_w = torch.empty(64 << 20, dtype=torch.uint8, device=dev)

    def timed(partition):
        def run():
            for _ in range(10):
                paged_attention(w["query"], w["key_cache"], w["value_cache"], w["block_tables"], w["context_lens"],
                                16, backend="hip", validate=False, partition_tokens=partition, out=wout,
                                workspace=ws_w)
        ms, _ = graph_time_ms(run, torch, calls_per_graph=10, replays=10, warmup=2)
        return ms / 10 * 1e-3
    split_call = timed(2048)
    walk_call = timed(0)
    rows = int(w["context_lens"].sum())
    nbytes = rows * 4096 + 2 * 16 * 16 * 128 * 2 + 16 * 512 * 8 + 16 * 8
    err = None if cpu is None else max_abs(wout, cpu.decode({k: w[k].cpu() for k in DECODE_NAMES}, 16))
    extra["ragged_b16_ctx8192_bf16_balanced_walk"] = {
        "us_per_call": walk_call * 1e6, "GBps": nbytes / walk_call / 1e9,
        "frac_of_hbm_peak": nbytes / walk_call / 1e9 / HBM_PEAK_GBS, "split_k_2048_us_per_call": split_call * 1e6,
        "rows": rows, "algorithmic_bytes": nbytes, "max_abs_error": err}


def _extra_shards(torch, paged_attention, cpu, dev, extra):
    """One GPU's share of the headline step under the sharding the path would
    use (nothing here runs a second GPU): kv heads split over 2 or 8 GPUs (4
    or 1 kv heads per GPU, with their query heads) or the sequences over 8
    GPUs (4 per GPU).  Each share runs over 28 separately allocated pools in
    one graph, as the headline step; layer 0 is checked against the oracle."""
    shards = {"tp2_kv_heads4": (BATCH, HQ // 2, HKV // 2), "tp8_kv_heads1": (BATCH, HQ // 8, HKV // 8),
              "dp8_batch4": (BATCH // 8, HQ, HKV)}
    gen = torch.Generator(device=dev).manual_seed(BASE_SEED + 300)
    width = CONTEXT // BLOCK
    result = {}
    for name, (batch, hq, hkv) in shards.items():
        pages = batch * width + 7
        layers = []
        for _ in range(LAYERS):
            layers.append({
                "query": torch.randn((batch, hq, D), generator=gen, device=dev).half(),
                "key_cache": torch.randn((pages, BLOCK, hkv, D), generator=gen, device=dev).half(),
                "value_cache": torch.randn((pages, BLOCK, hkv, D), generator=gen, device=dev).half(),
                "block_tables": torch.randperm(pages, generator=gen, device=dev)[:batch * width].view(batch, width)
                .contiguous(),
                "context_lens": torch.full((batch,), CONTEXT, dtype=torch.int64, device=dev)})
            layers[-1]["out"] = torch.empty_like(layers[-1]["query"])

        def step():
            for c in layers:
                paged_attention(*(c[k] for k in DECODE_NAMES), BLOCK, backend="hip", validate=False, out=c["out"])
        ms, _ = graph_time_ms(step, torch, calls_per_graph=LAYERS, replays=20, warmup=3)
        per_call = ms / LAYERS * 1e-3
        nbytes = batch * CONTEXT * hkv * D * 2 * 2 + 2 * batch * hq * D * 2 + batch * width * 8 + batch * 8
        err = None
        if cpu is not None:
            c = layers[0]
            err = max_abs(c["out"], cpu.decode({k: c[k].cpu() for k in DECODE_NAMES}, BLOCK))
        result[name] = {"batch": batch, "q_heads": hq, "kv_heads": hkv, "us_per_call": per_call * 1e6,
                        "GBps": nbytes / per_call / 1e9, "frac_of_hbm_peak": nbytes / per_call / 1e9 / HBM_PEAK_GBS,
                        "algorithmic_bytes": nbytes, "max_abs_error": err}
        del layers
    extra["decode_shards_b32_ctx2048_fp16_28layers"] = result


def _extra_prefill(torch, write_kv_cache_slots, paged_prefill_attention, workloads, cpu, dev, extra):
    # Chunked prefill: 8 x 128 new tokens after U[0,3968] prior, bf16, block 256.
    c = workloads.chunked_prefill_case(device=dev)
    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    write_kv_cache_slots(c["key_cache"], c["value_cache"], c["slot_mapping"], c["new_key"], c["new_value"],
                         backend="hip", validate=False)
    pargs = [c[n] for n in names]
    holder = {}

    def pf():
        holder["out"] = paged_prefill_attention(*pargs, 256, backend="hip", validate=False)

    def many5(n=10):
        def run():
            for _ in range(n):
                pf()
        return run
    ms, _ = graph_time_ms(many5(), torch, calls_per_graph=10, replays=10, warmup=2)
    per_call = ms / 10 * 1e-3
    flops = workloads.prefill_flops(c["priors"])
    kv_bytes = sum(p + 128 for p in c["priors"]) * 4096 + 2 * 1024 * 16 * 128 * 2
    err = None if cpu is None else max_abs(holder["out"], cpu.prefill(*[a.cpu() for a in pargs], 256, cast=False))
    # The call sits near the ridge point: its roofline time is the larger of
    # the MFMA time and the HBM time of its algorithmic work.
    bound_s = max(flops / (MFMA_BF16_PEAK_TFLOPS * 1e12), kv_bytes / (HBM_PEAK_GBS * 1e9))
    extra["chunked_prefill_8x128_bf16"] = {
        "us_per_call": per_call * 1e6, "TFLOPs": flops / per_call / 1e12,
        "frac_of_bf16_mfma_peak": flops / per_call / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "GBps": kv_bytes / per_call / 1e9, "frac_of_hbm_peak": kv_bytes / per_call / 1e9 / HBM_PEAK_GBS,
        "algorithmic_bytes": kv_bytes, "roofline_bound_us": bound_s * 1e6,
        "frac_of_roofline_time": bound_s / per_call, "flops": flops, "priors": c["priors"],
        "max_abs_error": err}


def _extra_prefill_cold(torch, write_kv_cache_slots, paged_prefill_attention, workloads, cpu, dev, extra):
    """The 8 x 128 chunked prefill with its inputs cold: 8 separately
    allocated workloads (same priors, different data; about 63 MB of K/V
    pages each, 500 MB together, twice the 256 MB Infinity Cache) are cycled
    in one graph, as the headline cycles 28 layer pools, so that no call finds
    its pages in the cache a previous call left them in.  One workspace,
    sized for the call, serves every call (what a layer loop does)."""
    from mini_engine_hip.kernels.prefill import paged_prefill_workspace_bytes

    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    priors = [2220, 601, 877, 1126, 1381, 3550, 2532, 347]
    cases = []
    for i in range(8):
        c = workloads.chunked_prefill_case(device=dev, seed=BASE_SEED + 40 + i, priors=priors)
        write_kv_cache_slots(c["key_cache"], c["value_cache"], c["slot_mapping"], c["new_key"], c["new_value"],
                             backend="hip", validate=False)
        cases.append([c[n] for n in names])
    q, kc = cases[0][0], cases[0][1]
    need = paged_prefill_workspace_bytes(len(priors), q.shape[0], q.shape[1], kc.shape[2], q.shape[2], 256,
                                         cases[0][5].shape[1], q.dtype)
    workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    outs = [None] * len(cases)

    def cycle():
        for i, pargs in enumerate(cases):
            outs[i] = paged_prefill_attention(*pargs, 256, backend="hip", validate=False, workspace=workspace)

    ms, _ = graph_time_ms(cycle, torch, calls_per_graph=len(cases), replays=10, warmup=2)
    per_call = ms / len(cases) * 1e-3
    flops = workloads.prefill_flops(priors)
    kv_bytes = sum(p + 128 for p in priors) * 4096 + 2 * 1024 * 16 * 128 * 2
    bound_s = max(flops / (MFMA_BF16_PEAK_TFLOPS * 1e12), kv_bytes / (HBM_PEAK_GBS * 1e9))
    errs = None
    if cpu is not None:
        errs = max(max_abs(outs[i], cpu.prefill(*[a.cpu() for a in cases[i]], 256, cast=False)) for i in (0, 7))
    extra["chunked_prefill_8x128_bf16_cold"] = {
        "us_per_call": per_call * 1e6, "TFLOPs": flops / per_call / 1e12,
        "frac_of_bf16_mfma_peak": flops / per_call / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "GBps": kv_bytes / per_call / 1e9, "frac_of_hbm_peak": kv_bytes / per_call / 1e9 / HBM_PEAK_GBS,
        "roofline_bound_us": bound_s * 1e6, "frac_of_roofline_time": bound_s / per_call,
        "workloads_cycled": len(cases), "distinct_kv_bytes": sum(a[1].numel() * 4 for a in cases),
        "max_abs_error_calls_0_and_7": errs}
    del cases, outs, workspace
    torch.cuda.empty_cache()


def _extra_prefill_shapes(torch, write_kv_cache_slots, paged_prefill_attention, workloads, dev, extra):
    """The same kernels on larger chunked-prefill shapes (bf16, block 256,
    Hq16/Hkv8/D128): how far the fraction of the MFMA peak rises once each CU
    has more than one short item to run.  Outputs are checked against the
    oracle by the GPU tests at smaller sizes, not here."""
    shapes = (("8x512_priors_U0_3968", 8, 512, [2220, 601, 877, 1126, 1381, 3550, 2532, 347]),
              ("32x256_priors_U0_3968", 32, 256, None),
              ("4x4096_causal", 4, 4096, [0, 0, 0, 0]),
              ("1x16384_causal", 1, 16384, [0]))
    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    rows = {}
    for name, seqs, new_tokens, priors in shapes:
        c = workloads.chunked_prefill_case(device=dev, num_seqs=seqs, new_tokens=new_tokens, priors=priors)
        write_kv_cache_slots(c["key_cache"], c["value_cache"], c["slot_mapping"], c["new_key"], c["new_value"],
                             backend="hip", validate=False)
        pargs = [c[n] for n in names]

        def run(n=3):
            for _ in range(n):
                paged_prefill_attention(*pargs, 256, backend="hip", validate=False)
        ms, _ = graph_time_ms(run, torch, calls_per_graph=3, replays=10, warmup=3)
        per_call = ms / 3 * 1e-3
        flops = workloads.prefill_flops(c["priors"], new_tokens=new_tokens)
        rows[name] = {"us_per_call": per_call * 1e6, "TFLOPs": flops / per_call / 1e12,
                      "frac_of_bf16_mfma_peak": flops / per_call / 1e12 / MFMA_BF16_PEAK_TFLOPS, "flops": flops}
        del c, pargs
        torch.cuda.empty_cache()
    extra["chunked_prefill_other_shapes_bf16"] = rows


def _extra_dense_prefill(torch, workloads, cpu, dev, extra):
    """Dense causal suffix prefill (prefill_attention): the reference's
    single-request path, Attention.forward passing transposed views of
    [tokens, heads, head_dim] tensors (native_qwen3.py:137-140), bf16,
    Hq16/Hkv8/D128.  Square prompts of 2048 and 8192 tokens (8192 is the
    reference CUDA kernel's limit) and 512 tokens after 3584; the 2048-token
    prompt is checked against the oracle."""
    from mini_engine_hip.kernels.prefill import prefill_attention

    shapes = (("square_2048", 0, 2048), ("square_8192", 0, 8192), ("suffix_512_after_3584", 3584, 512))
    rows = {}
    for name, start, tokens in shapes:
        gen = torch.Generator().manual_seed(BASE_SEED + tokens + start)
        context = start + tokens
        q_rows = torch.randn(tokens, HQ, D, generator=gen).to(torch.bfloat16).to(dev)
        k_rows = torch.randn(context, HKV, D, generator=gen).to(torch.bfloat16).to(dev)
        v_rows = torch.randn(context, HKV, D, generator=gen).to(torch.bfloat16).to(dev)
        q, k, v = (t.transpose(0, 1).unsqueeze(0) for t in (q_rows, k_rows, v_rows))
        holder = {}

        def run(n=3):
            for _ in range(n):
                holder["out"] = prefill_attention(q, k, v, "hip", query_start=start)
        ms, _ = graph_time_ms(run, torch, calls_per_graph=3, replays=10, warmup=3)
        per_call = ms / 3 * 1e-3
        flops = workloads.prefill_flops([start], new_tokens=tokens)
        row = {"us_per_call": per_call * 1e6, "TFLOPs": flops / per_call / 1e12,
               "frac_of_bf16_mfma_peak": flops / per_call / 1e12 / MFMA_BF16_PEAK_TFLOPS, "flops": flops}
        if name == "square_2048":
            row["max_abs_error"] = None if cpu is None else max_abs(
                holder["out"], cpu.dense_prefill(q.cpu(), k.cpu(), v.cpu(), query_start=start, cast=False))
        rows[name] = row
        del q, k, v, q_rows, k_rows, v_rows, holder
        torch.cuda.empty_cache()
    extra["dense_prefill_bf16"] = rows


def _extra_kv_scatter(torch, write_kv_cache_slots, workloads, cpu, dev, extra):
    """The KV scatter alone (write_kv_cache_slots): the chunked-prefill workload's
    1,024 new rows (bf16, block 256) and the B8 decode workload's 8 rows (bf16,
    block 16, 2048-page pool).  Algorithmic bytes per row: K and V read and
    written (4 x 2,048 B at Hkv 8 / D 128) plus the 8-byte slot."""
    cases = (("kv_scatter_prefill_1024_rows_bf16", workloads.chunked_prefill_case(device=dev), 100),
             ("kv_scatter_decode_b8_8_rows_bf16", workloads.decode_b8_with_scatter(dev), 100))
    for name, c, n in cases:
        kc, vc, slots, nk, nv = c["key_cache"], c["value_cache"], c["slot_mapping"], c["new_key"], c["new_value"]
        fn = lambda: write_kv_cache_slots(kc, vc, slots, nk, nv, backend="hip", validate=False)  # noqa: E731

        def many(run_fn=fn, count=n):
            def run():
                for _ in range(count):
                    run_fn()
            return run
        ms, _ = graph_time_ms(many(), torch, calls_per_graph=n, replays=20, warmup=3)
        rows = slots.numel()
        moved = rows * (4 * HKV * D * 2 + 8)
        per_call = ms / n * 1e-3
        flat_k = kc.view(-1, HKV, D)[slots].cpu()
        flat_v = vc.view(-1, HKV, D)[slots].cpu()
        extra[name] = {"us_per_call": per_call * 1e6, "GBps": moved / per_call / 1e9,
                       "frac_of_hbm_peak": moved / per_call / 1e9 / HBM_PEAK_GBS, "rows": rows,
                       "algorithmic_bytes": moved,
                       "rows_bit_exact": bool(torch.equal(flat_k, nk.cpu()) and torch.equal(flat_v, nv.cpu()))}
        del c


def _norm_rope_case(torch, dev, tokens, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(tokens, (HQ + 2 * HKV) * D, generator=gen) * 3).to(dtype)
    angles = torch.randn(tokens, D // 2, generator=gen) * 4
    c = {"qkv": qkv, "cos": angles.cos().to(dtype), "sin": angles.sin().to(dtype),
         "wq": (torch.rand(D, generator=gen) + 0.5).to(dtype), "wk": (torch.rand(D, generator=gen) + 0.5).to(dtype)}
    c = {k: v.to(dev) for k, v in c.items()}
    c["q"] = c["qkv"][:, :HQ * D].view(tokens, HQ, D)
    c["k"] = c["qkv"][:, HQ * D:(HQ + HKV) * D].view(tokens, HKV, D)
    c["v"] = c["qkv"][:, (HQ + HKV) * D:].view(tokens, HKV, D)
    return c


def _extra_norm_rope(torch, cpu_leg, dev, extra):
    """Fused q/k RMSNorm + RoPE + KV write at the prefill batch (1024 tokens, bf16, block 256, slot
    mapping) and the decode batch (32 sequences, fp16, block 256, tables + positions), beside the same
    four steps as separate eager torch ops plus the HIP scatter (the reference's torch data path, timed
    eagerly on the stream, not captured)."""
    from mini_engine_hip.kernels.rope import qk_norm_rope_write_kv
    from mini_engine_hip.kernels.linear import linear_rows
    from mini_engine_hip.kernels.data import write_kv_cache_slots

    for name, tokens, dtype, mode in (("norm_rope_kv_write_prefill_1024tok_bf16", 1024, torch.bfloat16, "slots"),
                                      ("norm_rope_kv_write_decode_b32_fp16", 32, torch.float16, "tables")):
        c = _norm_rope_case(torch, dev, tokens, dtype, seed=BASE_SEED + tokens)
        pages = 300                   # distinct pages for every decode sequence (32 x 8 table entries)
        gen = torch.Generator().manual_seed(BASE_SEED + 7)
        kc = torch.randn(pages, BLOCK, HKV, D, generator=gen).to(dtype).to(dev)
        vc = torch.randn(pages, BLOCK, HKV, D, generator=gen).to(dtype).to(dev)
        slots = torch.randperm(pages * BLOCK, generator=gen)[:tokens].to(dev)
        meta = {"slot_mapping": slots}
        if mode == "tables":
            width = 8
            tables = torch.randperm(pages, generator=gen)[:tokens * width].view(tokens, width).to(dev)
            positions = torch.randint(0, width * BLOCK, (tokens,), generator=gen).to(dev)
            meta = {"block_tables": tables, "positions": positions}
            flat = (tables.gather(1, (positions // BLOCK)[:, None])[:, 0] * BLOCK + positions % BLOCK)
            slots = flat
        out = torch.empty(tokens, HQ, D, dtype=dtype, device=dev)
        args = (c["q"], c["k"], c["v"], c["wq"], c["wk"], c["cos"], c["sin"], kc, vc)
        fused = lambda: qk_norm_rope_write_kv(*args, validate=False, out=out, **meta)  # noqa: E731

        def eager_four_steps():
            q = c["q"].float()
            q = (q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype) * c["wq"]
            k = c["k"].float()
            k = (k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype) * c["wk"]
            cs, sn, half = c["cos"].unsqueeze(1), c["sin"].unsqueeze(1), D // 2
            q = torch.cat((q[..., :half] * cs - q[..., half:] * sn, q[..., :half] * sn + q[..., half:] * cs), -1)
            k = torch.cat((k[..., :half] * cs - k[..., half:] * sn, k[..., :half] * sn + k[..., half:] * cs), -1)
            write_kv_cache_slots(kc, vc, slots, k, c["v"], backend="hip", validate=False)
            return q

        def many(fn, n):
            def run():
                for _ in range(n):
                    fn()
            return run
        ms, _ = graph_time_ms(many(fused, 50), torch, calls_per_graph=50, replays=20, warmup=3)
        eager_four_steps()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        many(eager_four_steps, 10)()
        end.record()
        end.synchronize()
        eager_ms = start.elapsed_time(end)
        per_call = ms / 50 * 1e-3
        moved = (tokens * (HQ + 2 * HKV) * D * 2 + tokens * D * 2 + 2 * D * 2 + tokens * 8 * (2 if mode == "tables"
                 else 1) + tokens * HQ * D * 2 + tokens * 2 * HKV * D * 2)
        extra[name] = {
            "us_per_call": per_call * 1e6, "GBps": moved / per_call / 1e9,
            "frac_of_hbm_peak": moved / per_call / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": moved,
            "eager_torch_four_steps_us": eager_ms / 10 * 1e3,
            "q_max_abs_error": None, "q_bit_identical_frac": None, "k_max_abs_error": None, "v_bit_exact": None}
        if cpu_leg is not None:
            # The last call against the reference (q rows; written K rows; V rows bit-exact).
            fused()
            torch.cuda.synchronize()
            cpu = {k: v.cpu() for k, v in c.items()}
            kc_o = torch.zeros(pages, BLOCK, HKV, D, dtype=dtype)
            vc_o = torch.zeros(pages, BLOCK, HKV, D, dtype=dtype)
            cpu_meta = {k: v.cpu() for k, v in meta.items()}
            want_q = cpu_leg.norm_rope_write_kv(cpu["q"], cpu["k"], cpu["v"], cpu["wq"], cpu["wk"], cpu["cos"],
                                                cpu["sin"], kc_o, vc_o, **cpu_meta)
            rows = slots.cpu()
            got_k, want_k = kc.cpu().view(-1, HKV, D)[rows], kc_o.view(-1, HKV, D)[rows]
            extra[name].update({
                "q_max_abs_error": max_abs(out, want_q),
                "q_bit_identical_frac": (out.cpu() == want_q).float().mean().item(),
                "k_max_abs_error": max_abs(got_k, want_k),
                "v_bit_exact": bool(torch.equal(vc.cpu().view(-1, HKV, D)[rows], vc_o.view(-1, HKV, D)[rows]))})


def _extra_after_attention(torch, cpu, dev, extra):
    """The step after attention at the headline batch: the o_proj projection of 32 rows over 28
    layers' distinct weights (the reference's CudaLinear -- torch.mm(x, weight.t()) on the
    [out, in] weight, a library GEMM -- beside mvme_linear_rows, HipLinear's decode-batch kernel)
    and greedy argmax over a 151,936-entry vocabulary (the HIP kernel), 32 sequences, hidden 2048."""
    from mini_engine_hip.sampling import greedy_argmax
    from mini_engine_hip.kernels.linear import linear_rows

    batch, hidden, vocab = BATCH, 2048, 151936
    gen = torch.Generator().manual_seed(BASE_SEED + 11)
    attn = torch.randn(batch, HQ * D, generator=gen).to(torch.bfloat16).to(dev)
    dgen = torch.Generator(device=dev).manual_seed(BASE_SEED + 12)
    weights = [(torch.randn(hidden, HQ * D, generator=dgen, device=dev) * 0.02).to(torch.bfloat16)
               for _ in range(LAYERS)]  # o_proj.weight of each layer, [out, in]
    out_lib = torch.empty(batch, hidden, dtype=torch.bfloat16, device=dev)
    out_hip = torch.empty(batch, hidden, dtype=torch.bfloat16, device=dev)

    def many(fn, n):
        def run():
            for _ in range(n):
                fn()
        return run

    def layers(fn):
        def run():
            for w in weights:
                fn(w)
        return run
    ms_lib, _ = graph_time_ms(layers(lambda w: torch.mm(attn, w.t(), out=out_lib)), torch, calls_per_graph=LAYERS,
                              replays=20, warmup=3)
    ms_hip, _ = graph_time_ms(layers(lambda w: linear_rows(attn, w, out=out_hip)), torch, calls_per_graph=LAYERS,
                              replays=20, warmup=3)
    o_bytes = HQ * D * hidden * 2 + batch * HQ * D * 2 + batch * hidden * 2
    o_ref = attn.float().cpu() @ weights[-1].float().cpu().t()
    per_hip, per_lib = ms_hip / LAYERS * 1e-3, ms_lib / LAYERS * 1e-3
    extra["o_proj_b32_2048x2048_bf16_28_weights"] = {
        "us_per_call": per_hip * 1e6, "GBps": o_bytes / per_hip / 1e9,
        "frac_of_hbm_peak": o_bytes / per_hip / 1e9 / HBM_PEAK_GBS,
        "kernel": "mvme_linear_rows", "max_abs_error_vs_fp32": max_abs(out_hip, o_ref),
        "library_torch_mm_us_per_call": per_lib * 1e6, "library_max_abs_error_vs_fp32": max_abs(out_lib, o_ref)}
    del weights
    for dtype, name in ((torch.bfloat16, "greedy_argmax_b32_vocab151936_bf16"),
                        (torch.float32, "greedy_argmax_b32_vocab151936_fp32")):
        logits = torch.randn(batch, vocab, generator=gen).to(dtype).to(dev)
        tokens = torch.empty(batch, dtype=torch.int64, device=dev)
        ms, _ = graph_time_ms(many(lambda: greedy_argmax(logits, out=tokens), 50), torch, calls_per_graph=50,
                              replays=20, warmup=3)
        moved = batch * vocab * logits.element_size() + batch * 8
        extra[name] = {"us_per_call": ms / 50 * 1e3, "GBps": moved / (ms / 50 * 1e-3) / 1e9,
                       "frac_of_hbm_peak": moved / (ms / 50 * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "tokens_equal_reference": None if cpu is None else
                       bool(torch.equal(tokens.cpu(), cpu.greedy(logits.cpu())))}


def summarize_headline_trace(path, steps, warmup):
    """Average duration of the headline decode kernel over the timed graph replays.

    In a headline-only run, headline() dispatches the 28 layer calls once
    eagerly (before capture), then `warmup` untimed replays, then the `steps`
    timed replays, then 4 eager repetitions for the wall-clock figure; the
    timed dispatches are therefore positions [28 (1 + warmup), 28 (1 + warmup
    + steps)) of the decode kernel's dispatches in start-time order."""
    import csv

    with open(path, newline="") as f:
        rows = [r for r in csv.DictReader(f) if "paged_decode_kernel" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    first, last = LAYERS * (1 + warmup), LAYERS * (1 + warmup + steps)
    if len(rows) < last:
        raise SystemExit(f"{path}: {len(rows)} decode dispatches, expected at least {last}")
    timed = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows[first:last]]
    every = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows]
    span = (int(rows[last - 1]["End_Timestamp"]) - int(rows[first]["Start_Timestamp"])) / 1e3
    return {"kernel": rows[first]["Kernel_Name"][:96], "dispatches": len(rows), "timed_dispatches": len(timed),
            "timed_avg_us": statistics.mean(timed), "timed_min_us": min(timed), "timed_max_us": max(timed),
            "timed_avg_x28_ms": statistics.mean(timed) * LAYERS / 1e3,
            "timed_span_per_step_ms": span / steps / 1e3, "all_avg_us": statistics.mean(every)}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--partition", type=int, default=0, help="split-K partition tokens (0 = library default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--extra", default=",".join(EXTRA_NAMES),
                    help="comma-separated subset of the other workloads: " + ",".join(EXTRA_NAMES))
    ap.add_argument("--no-headline", action="store_true", help="skip the headline decode (profiling runs)")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-baseline timing")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 plain 1 GiB device copies (scale reference for HBM byte counters)")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="summarise a rocprofv3 kernel trace of a headline-only run (--no-extra) made with the "
                         "same --steps/--warmup: the headline kernel's average over the timed replays only")
    args = ap.parse_args(argv)
    if args.trace_summary:
        print(json.dumps(summarize_headline_trace(args.trace_summary, args.steps, args.warmup)))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the paged-attention path runs on a single MI355X and "
              f"--gpus {args.gpus} is not supported (decode would shard by sequence or kv head with no "
              f"exchange; this benchmark does not launch ranks)", file=sys.stderr)
        return 2

    import torch

    from mini_engine_hip.kernels import hip_extension
    from mini_engine_hip.kernels.data import write_kv_cache_batch, write_kv_cache_slots
    from mini_engine_hip.kernels.paged import paged_attention
    from mini_engine_hip.kernels.prefill import paged_prefill_attention
    from mini_engine_hip import workloads

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    if args.copy_calibration:
        src = torch.ones(1 << 29, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": src.numel() * 2, "copy_calibration_bytes_written":
                          dst.numel() * 2, "copies": 10}))
        return 0
    lib = hip_extension.load_hip_extension()
    log(f"library {lib.path}")
    # The CPU leg (timed reference path and checker); nothing else uses the oracle.
    cpu = None if args.no_cpu_baseline else CpuLeg(torch)
    if args.no_headline:
        extra = extra_workloads(torch, paged_attention, write_kv_cache_slots, paged_prefill_attention, workloads,
                                cpu, names=tuple(args.extra.split(",")))
        print(json.dumps({"profiling_run": True, "extra": extra}), flush=True)
        return 0

    layers, step_ms, eager_ms = headline(args, torch, paged_attention, workloads)
    per_call_ms = step_ms / LAYERS
    step_bytes = LAYERS * layer_bytes()
    achieved_gbs = layer_bytes() / (per_call_ms * 1e-3) / 1e9
    log(f"headline: {step_ms:.3f} ms/step, {per_call_ms * 1e3:.2f} us/call, {achieved_gbs:.0f} GB/s")
    parity = None if cpu is None else headline_parity(layers, cpu)
    log(f"parity: {parity}")
    decode_step = attention_block = None
    if not args.no_extra:
        decode_step = decode_step_with_scatter(args, torch, layers, write_kv_cache_batch, paged_attention, cpu)
        log(f"decode step with scatter: {decode_step}")
        attention_block = decode_attention_block_step(args, torch, layers, paged_attention, cpu)
        log(f"decode attention block: {attention_block}")

    traffic = None
    traffic_file = ROOT / "profiles" / "paged_decode_b32_ctx2048_traffic.txt"
    if traffic_file.exists():
        for line in traffic_file.read_text().splitlines():
            if line.startswith("hbm_bytes_per_launch:"):
                traffic = int(line.split(":", 1)[1])

    result = {
        "metric": METRIC,
        "value": step_bytes / (step_ms * 1e-3) / 1e12,
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "us_per_call": per_call_ms * 1e3,
        "eager_wall_us_per_call": eager_ms / LAYERS * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1) q/K/V, seeded random non-contiguous pages; inputs resident in HBM",
        "config": {"workload": "paged_decode_b32_ctx2048_fp16_block256_28layers", "batch": BATCH,
                   "context": CONTEXT, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "block_size": BLOCK,
                   "layers": LAYERS, "kv_pool_per_layer": "263 pages, separate per layer",
                   "algorithmic_bytes_per_call": layer_bytes(), "timing": "hipGraph of 28 calls per step"},
        "roofline": {"bound": "hbm", "achieved": achieved_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved_gbs / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": "paged_decode_kernel (fp16, D=128, G=2, 8 waves)"},
        "parity": parity,
        "reference_published": {"us_per_call_rtx5080": REFERENCE_US_PER_CALL,
                                "speedup_vs_rtx5080": REFERENCE_US_PER_CALL / (per_call_ms * 1e3)},
    }
    del layers
    torch.cuda.empty_cache()
    if not args.no_extra:
        result["extra"] = extra_workloads(torch, paged_attention, write_kv_cache_slots, paged_prefill_attention,
                                          workloads, cpu, names=tuple(args.extra.split(",")))
        result["extra"]["decode_step_b32_ctx2048_28layers_with_scatter"] = decode_step
        result["extra"]["decode_attention_block_b32_ctx2048_28layers"] = attention_block
        log(f"extra: {json.dumps(result['extra'])}")
    if cpu is not None:
        result["cpu_baseline"] = cpu.baseline(workloads, args.cpu_budget)
        log(f"cpu baseline: {result['cpu_baseline']}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
