"""Headline benchmark: BF16-in / F32-accumulate C = A.B at 4096^3 on one MI355X.

BASELINE.json's metric is "matmul TFLOP/s (% MFMA peak) + SmolLM2-135M-shape
decoder tokens/sec, 1 GPU"; its matmul configuration (configs[1], the cube
sweep) at its target size, bf16 4096^3, is the workload of `value`.  A step is
one product of two resident [4096, 4096] BF16 matrices into a fresh F32 result
through the C ABI (`mi_matmul`), inputs already in HBM.

Printed: one JSON line with `value` (TFLOP/s over the timed steps, wall clock
with a stream sync on both sides), the kernel's roofline (achieved TFLOP/s
from HIP events recorded on the engine's own stream around the timed steps,
against MI355X's dense BF16 peak), and the CPU baseline (the oracle's F32
product timed on this host's cores: the same 4096^3 product repeated for
about 10 s).

The same line carries BASELINE.json's other measured configs: `decoder`, the
SmolLM2-135M-shaped decoder (config 5) at batch 1 and 32 -- prefill 512 tokens,
greedy-decode 128, tokens/s, under the reference numeric contract and (in
`decoder_performance_numerics`) the performance one -- and `mlp_train`, the MLP training step
(config 1), ms/step over 100 steps.

Before the timed steps the product runs untimed for the W warm-up steps and
at least two seconds (the GPU's clocks ramp up under sustained load; the
timed steps measure the steady state).

Flags: --gpus N (only 1: this build runs on one GPU), --steps K, --warmup W,
--n (cube size, default 4096), --dtype bf16|f32, --no-cpu, --no-models.  `--suite` instead
prints one JSON line per kernel of the HBM-bound suite (BASELINE.json
configs[2]) and the matmul sweep, each against its roofline.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "metalium-rs_amd"))

PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}  # MI355X dense MFMA (AMD published)
HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the bf16 4096^3 NN product, from two rocprofv3 --pmc
# passes over `bench.py --no-cpu --no-models --steps 5 --warmup 1` (FETCH_SIZE,
# then WRITE_SIZE, KiB per dispatch), each scaled by what the counter reads for
# a plain copy of 256 MiB (FETCH_SIZE x 1.9998, WRITE_SIZE x 1.0): 196,904 KiB
# read + 65,536 KiB written.  Only that configuration was measured.
GEMM_TRAFFIC_BYTES = {("bf16", 4096): 268738874}
WARM_S = 2.0  # seconds of untimed product before the timed steps (clock ramp-up)


def cpu_baseline(n: int = 4096, seconds: float = 10.0) -> dict:
    """The oracle's F32 product (k ascending, F32 accumulation; register tiles
    of 4 x 32, AVX-512 / AVX2 clones, OpenMP over column strips) on this
    host's cores: the CPU restatement standing in for burn-flex, which cannot
    be built here.  The sample is the headline's own shape, repeated for
    about `seconds` of CPU work."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc
    cores = _cpu_cores()
    rng = np.random.default_rng(1)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    orc.matmul_f32acc(a[:64], b, threads=cores)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.matmul_f32acc(a, b, threads=cores)
        reps += 1
        el = time.perf_counter() - t0
        if el > seconds:
            break
    tflops = 2.0 * n ** 3 * reps / el / 1e12
    return {"value": round(tflops, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle F32 product {n}^3 (k-ascending F32 sums, 4x32 register tiles, vector ISA "
                      f"clones, OpenMP column strips), {reps} reps in {el:.2f} s"}


def _cpu_cores() -> int:
    """The host cores this process may run on (sched_getaffinity), within the
    CPU share its environment grants (OMP_NUM_THREADS, when set: 16 on the
    MI355X boxes these numbers come from)."""
    n = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(share)) if share.isdigit() and int(share) > 0 else n


def cpu_models_baseline() -> dict:
    """The reference's model workloads on this host's cores, in the float32
    torch restatements the device harnesses are checked against
    (oracle/models_cpu.py), standing in for burn-flex (not buildable here).
    Bounded samples of each workload, 10 to 30 s of CPU work in all."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch
    import models_cpu as mc
    import miburn
    cores = _cpu_cores()
    torch.set_num_threads(cores)
    out = {}
    kind = {"unit": "ms", "cores": cores, "kind": "port"}
    # Config 1: MLP 784-128-10, batch 64, SGD lr 0.01, fresh batches.
    g = torch.Generator().manual_seed(0)
    ps = [torch.empty(784, 128).uniform_(-1 / 28, 1 / 28, generator=g).requires_grad_(),
          torch.empty(128).uniform_(-1 / 28, 1 / 28, generator=g).requires_grad_(),
          torch.empty(128, 10).uniform_(-0.088, 0.088, generator=g).requires_grad_(),
          torch.empty(10).uniform_(-0.088, 0.088, generator=g).requires_grad_()]
    data = [(torch.rand(64, 784, generator=g), torch.randint(0, 10, (64,), generator=g)) for _ in range(110)]
    for i, (x, y) in enumerate(data):
        if i == 10:
            t0 = time.perf_counter()
        mc.mlp_loss(ps, x, y).backward()
        mc.sgd(ps, 0.01)
    ms = (time.perf_counter() - t0) * 1e3 / 100
    out["mlp_train"] = dict(value=round(ms, 4), **kind, sample="torch CPU float32 restatement, 100 SGD steps "
                            "(after 10 warm), batch 64")
    # Config 4: the transformer training step at its shape.
    cfg = miburn.TRANSFORMER_CONFIG4
    P, layers = mc.transformer_init(cfg, seed=0)
    every = list(P.values()) + [t for L in layers for t in L.values()]
    toks = [(torch.randint(0, cfg["vocab"], (16, 128), generator=g).numpy(),
             torch.randint(0, cfg["vocab"], (16, 128), generator=g).numpy()) for _ in range(3)]
    for i, (x, y) in enumerate(toks):
        if i == 1:
            t0 = time.perf_counter()
        mc.transformer_loss(P, layers, cfg, x, y).backward()
        mc.sgd(every, 0.05)
    ms = (time.perf_counter() - t0) * 1e3 / 2
    out["transformer_train"] = dict(value=round(ms, 2), **kind, sample="torch CPU float32 restatement, 2 "
                                    "forward + backward + SGD steps (after 1 warm), batch 16 x 128 tokens")
    # Config 5: the SmolLM2-shaped decoder (BF16-rounded N(0, 0.02) weights
    # held in F32), greedy decoding through a KV cache.
    lc = miburn.SMOLLM2_135M
    W = mc.llama_random_weights(lc, seed=0)
    with torch.no_grad():
        ids = torch.randint(0, lc["vocab"], (32, 512), generator=g).numpy()
        mc.llama_generate(W, lc, ids[:1, :16], 2)  # warm
        _, pf1, dc1 = mc.llama_generate(W, lc, ids[:1], 17, max_ctx=640)
        # Batch 32: the prefill of 2 of the 32 sequences (a CPU at full width
        # already: tokens/s scale with the batch), and decode steps at batch
        # 32 after a 512-position cache (its contents do not change the time).
        t0 = time.perf_counter()
        mc.llama_step(W, lc, mc.LlamaCache(lc, 2, 513), ids[:2])
        pf2 = (time.perf_counter() - t0) * 1e3
        cache = mc.LlamaCache(lc, 32, 640)
        cache.len = 512
        nxt = ids[:, :1]
        mc.llama_step(W, lc, cache, nxt)  # warm
        t0 = time.perf_counter()
        for _ in range(4):
            h = mc.llama_step(W, lc, cache, nxt)
            nxt = mc.argmax_first(h[:, -1] @ W["embed"].T)[:, None].numpy()
        dc32 = (time.perf_counter() - t0) * 1e3 / 4
    out["decoder_b1"] = {"prefill_tokens_per_s": round(512 / (pf1 / 1e3), 1),
                         "decode_ms_per_step": round(dc1 / 16, 3), "decode_tokens_per_s": round(16 / (dc1 / 1e3), 1),
                         "cores": cores, "kind": "port",
                         "sample": "torch CPU float32 restatement: 512-token prefill, 16 greedy steps"}
    out["decoder_b32"] = {"prefill_tokens_per_s": round(2 * 512 / (pf2 / 1e3), 1),
                          "decode_ms_per_step": round(dc32, 3), "decode_tokens_per_s": round(32 / (dc32 / 1e3), 1),
                          "cores": cores, "kind": "port",
                          "sample": "torch CPU float32 restatement: 512-token prefill of 2 sequences, 4 greedy "
                                    "steps at batch 32 after 512 cached positions"}
    return out


def _time_op(eng, fn, reps: int, warm: int = 3) -> float:
    """Average device time (ms) of `fn` (which returns an id to free), from
    HIP events on the engine's stream.  Each result is freed as soon as it is
    made: the engine's caching allocator hands the same block to the next call
    (one stream orders every use), so no allocation stalls the timed region."""
    for _ in range(warm):
        eng.free(fn())
    eng.sync()
    eng.event_record(2)
    for _ in range(reps):
        eng.free(fn())
    eng.event_record(3)
    return eng.event_elapsed_ms(2, 3) / reps


def suite(steps: int, matmul_mode=None) -> int:
    """HBM-bound kernels on [8192, 8192] F32 and the
    matmul cube sweep: one JSON line per kernel."""
    import miburn
    eng = miburn.Engine(0)
    if matmul_mode:
        eng.set_matmul_mode(miburn.MATMUL_FAST if matmul_mode == "fast" else miburn.MATMUL_ACCURATE)
    R = C = 8192
    n = R * C
    x = eng.random_dram(R, C, miburn.DRAW_NORMAL, 0.0, 1.0, base=21)
    y = eng.random_dram(R, C, miburn.DRAW_NORMAL, 0.0, 1.0, base=22)
    reps = max(5, steps // 10)
    lines = []

    def hbm(name, fn, nbytes):
        ms = _time_op(eng, fn, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        lines.append({"kernel": name, "config": "f32 [8192, 8192]" if "gather" not in name else
                      "table [49152, 576] f32, 65536 ids", "ms": round(ms, 5), "bytes": nbytes,
                      "achieved_GBs": round(gbs, 1), "peak_GBs": HBM_PEAK_GBS, "frac": round(gbs / HBM_PEAK_GBS, 4)})

    # A plain device copy of one operand (hipMemcpyAsync): the reference the
    # PMC traffic counters are scaled by (its bytes are known exactly).
    def copy():
        eng.copy_into(x, y)
        return eng.empty(1, 1)
    hbm("copy (calibration)", copy, 8 * n)
    hbm("add", lambda: eng.eltwise_op_as("ADD", x, y), 12 * n)
    hbm("mul", lambda: eng.eltwise_op_as("MUL", x, y), 12 * n)
    for k in ("EXP", "GELU", "SILU"):
        hbm(k.lower(), lambda k=k: eng.eltwise_op_as(k, x), 8 * n)
    hbm("rsqrt(|x|+1e-6) fused", lambda: eng.eltwise_op_as("RSQRT_ABS_ADD", x, scalar=1e-6), 8 * n)
    hbm("row softmax", lambda: eng.softmax_rows(x), 8 * n)
    hbm("row sum (dim 1)", lambda: eng.reduce(x, miburn.R_SUM, miburn.AXIS_COLS), 4 * n + 4 * R)
    hbm("row mean (dim 1)", lambda: eng.reduce(x, miburn.R_MEAN, miburn.AXIS_COLS), 4 * n + 4 * R)
    hbm("column sum (dim 0)", lambda: eng.reduce(x, miburn.R_SUM, miburn.AXIS_ROWS), 4 * n + 4 * C)
    hbm("column mean (dim 0)", lambda: eng.reduce(x, miburn.R_MEAN, miburn.AXIS_ROWS), 4 * n + 4 * C)
    eng.free(x)
    eng.free(y)
    table = eng.random_dram(49152, 576, miburn.DRAW_NORMAL, 0.0, 1.0, base=23)
    ids = eng.random_dram(1, 65536, miburn.DRAW_INT_RANGE, 0, 49152, base=24)
    hbm("embedding gather", lambda: eng.select_rows(table, ids), 2 * 65536 * 576 * 4 + 65536 * 4)
    for line in lines:
        print(json.dumps(line), flush=True)

    for dt in ("bf16", "f32"):
        for m in (512, 1024, 2048, 4096, 8192):
            a = eng.random_dram(m, m, miburn.DRAW_NORMAL, 0.0, 1.0, base=31)
            b = eng.random_dram(m, m, miburn.DRAW_NORMAL, 0.0, 1.0, base=32)
            if dt == "bf16":
                a2, b2 = eng.cast_float(a, miburn.BF16), eng.cast_float(b, miburn.BF16)
                eng.free(a)
                eng.free(b)
                a, b = a2, b2
            r = max(3, min(reps, int(2e12 / (2 * m ** 3)) + 3))
            ms = _time_op(eng, lambda: eng.matmul_dram(a, False, b, False), r)
            tf = 2 * m ** 3 / (ms * 1e-3) / 1e12
            print(json.dumps({"kernel": f"matmul {dt}", "config": f"{m}^3 NN", "ms": round(ms, 5),
                              "achieved_TFLOPs": round(tf, 1), "peak_TFLOPs": PEAK_TFLOPS[dt],
                              "frac": round(tf / PEAK_TFLOPS[dt], 4)}), flush=True)
            eng.free(a)
            eng.free(b)
        a = eng.random_dram(16 * 512, 512, miburn.DRAW_NORMAL, 0.0, 1.0, base=33)
        b = eng.random_dram(16 * 512, 512, miburn.DRAW_NORMAL, 0.0, 1.0, base=34)
        if dt == "bf16":
            a, b = eng.cast_float(a, miburn.BF16), eng.cast_float(b, miburn.BF16)
        ms = _time_op(eng, lambda: eng.matmul_dram_batched(a, False, b, False, 16, 512, 512, 512), reps)
        tf = 16 * 2 * 512 ** 3 / (ms * 1e-3) / 1e12
        print(json.dumps({"kernel": f"batched matmul {dt}", "config": "[16,512,512]x[16,512,512]",
                          "ms": round(ms, 5), "achieved_TFLOPs": round(tf, 1), "peak_TFLOPs": PEAK_TFLOPS[dt],
                          "frac": round(tf / PEAK_TFLOPS[dt], 4)}), flush=True)
    eng.close()
    return 0


def decoder_bench(eng, batch: int, prompt: int = 512, new: int = 128, numerics: str = "reference",
                  traced: bool = True) -> dict:
    """the SmolLM2-135M-shaped decoder (random N(0, 0.02)
    BF16 weights), prefill `prompt` random tokens per sequence, then greedy
    decode `new` tokens; tokens/s of the prefill and of the decode steps.
    `numerics`: the reference contract (F32 KV cache and activations) or the
    performance one (BFP8 projection weights, BF16 KV cache, BF16 prefill
    activation operands).  The generation runs eagerly (after an untimed one
    of the same prompt, so the allocator's blocks exist), then traced (the
    prompt's prefill and each decode step replays of captures -- the step per
    64-position span, chained on the device: each replay's tokens are the
    next one's input, read back once at the end -- the reference's
    TracedGenerator); the traced run's captures are made by an untimed first
    traced generation, and its tokens must be the eager ones.
    `traced` False skips the traced runs (profiling: rocprofv3's kernel
    trace has ended in a host segmentation fault inside hipGraphLaunch)."""
    import miburn
    m = miburn.Llama(eng, miburn.SMOLLM2_135M, max_ctx=prompt + new, max_batch=batch, seed=5, numerics=numerics)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 49152, (batch, prompt)).astype(np.int32)
    m.generate(ids, 4)  # warm the kernels and the allocator at the measured shapes
    out, pf_ms, dc_ms = m.generate(ids, new)
    tr_ms = tr_pf = None
    if traced:
        m.generate(ids, new, traced=True)  # captures the prompt's prefill and every span's step
        tr_out, tr_pf, tr_ms = m.generate(ids, new, traced=True)
        if not np.array_equal(tr_out, out):
            raise RuntimeError("traced generation's tokens differ from the eager loop's")
    m.close()
    # Rooflines (algorithmic work): a decode step reads every weight once
    # (134.48 M parameters, the tied table included: BF16, 2 B each; under
    # the performance contract the layers' 106.17 M are BFP8, 1 + 1/16 B
    # each, and the table stays BF16) plus each sequence's
    # key/value cache (2 x 30 layers x 3 kv heads x 64 x 4 B a position for
    # F32, 2 B for BF16, at the steps' mean context); a prefill's FLOP are
    # 2 x tokens x the layers'
    # 106.17 M weights plus causal attention (2 t (t + 1) x 64 x 9 heads x 30
    # layers a sequence) and the last position's head.
    cfg = miburn.SMOLLM2_135M
    per_layer = ((cfg["heads"] + 2 * cfg["kv_heads"]) * cfg["head_dim"] * cfg["hidden"] + cfg["hidden"] ** 2
                 + 3 * cfg["intermediate"] * cfg["hidden"])
    layer_params = cfg["layers"] * per_layer
    params = layer_params + cfg["vocab"] * cfg["hidden"]
    kv_per_pos = 2 * cfg["layers"] * cfg["kv_heads"] * cfg["head_dim"] * (2 if numerics == "performance" else 4)
    mean_ctx = prompt + new / 2
    weight_bytes = (layer_params * 17 / 16 + 2 * cfg["vocab"] * cfg["hidden"]) if numerics == "performance" \
        else 2 * params
    step_bytes = weight_bytes + batch * kv_per_pos * mean_ctx
    dc_step_ms = dc_ms / max(new - 1, 1)
    attn = 2 * prompt * (prompt + 1) * cfg["head_dim"] * cfg["heads"] * cfg["layers"]
    pf_flop = batch * (2 * prompt * layer_params + attn + 2 * cfg["hidden"] * cfg["vocab"])
    return {"batch": batch, "numerics": numerics, "prompt": prompt, "new_tokens": new,
            "prefill_ms": round(pf_ms, 2), "prefill_traced_ms": round(tr_pf, 2) if traced else None,
            "prefill_tokens_per_s": round(batch * prompt / (pf_ms / 1e3), 1),
            "prefill_gflop": round(pf_flop / 1e9, 1),
            "prefill_mfma_frac": round(pf_flop / (pf_ms * 1e-3) / (PEAK_TFLOPS["bf16"] * 1e12), 4),
            "decode_ms_per_step": round(dc_step_ms, 3),
            "decode_traced_ms_per_step": round(tr_ms / max(new - 1, 1), 3) if traced else None,
            "decode_tokens_per_s": round(batch * (new - 1) / (dc_ms / 1e3), 1),
            "decode_hbm_mb_per_step": round(step_bytes / 1e6, 1),
            "decode_hbm_frac": round(step_bytes / (dc_step_ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)}


def traced_steps(eng, step_ids, inputs, batches):
    """Capture one training step (`step_ids()` on the resident `inputs`), then
    replay it once per host batch, each overwriting the inputs (the reference's
    traced training loop, crates/tt-mnist/src/transformer.rs:177-230): ms per
    step with the batches uploaded inside the timed region, and ms per replay
    of the graph alone (inputs left resident)."""
    eng.begin_trace()
    loss = step_ids()
    trace = eng.end_trace()
    eng.run_trace(trace, dict(zip(inputs, batches[0])))  # warm
    eng.sync()
    t0 = time.perf_counter()
    for b in batches:
        eng.run_trace(trace, dict(zip(inputs, b)))
    eng.sync()
    t1 = time.perf_counter()
    for _ in batches:
        eng.run_trace(trace)
    eng.sync()
    t2 = time.perf_counter()
    eng.release_trace(trace)
    eng.free(loss)
    return (t1 - t0) * 1e3 / len(batches), (t2 - t1) * 1e3 / len(batches)


def decode_layer_bench(eng, batch: int = 1, ctx: int = 576, steps: int = 200) -> dict:
    """One SmolLM2-135M layer's decode launches alone, for counter profiles
    (rocprofv3 --pmc of the whole decoder harness has ended in host
    segmentation faults inside the profiler): the fused norm + q|k|v +
    attention step at a `ctx`-position context through the o projection and
    residual (mi_norm_qkv_attention_o: its chunk kernel, then the combine and
    the o projection -- one launch for one sequence), then the gate|up and
    down GEMVs (mi_norm_matvec) -- the launches of a decode layer as the model
    runs them (crates/tt-models/src/llama.rs:380-520) -- `steps` times over
    one layer's random BF16 weights and a random F32 cache."""
    import miburn
    H, KVH, D, hid, inter, maxc = 9, 3, 64, 576, 1536, 1024

    def bf(r, c, base):
        t = eng.random_dram(r, c, miburn.DRAW_NORMAL, 0.0, 0.02, base=base)
        y = eng.cast_float(t, miburn.BF16)
        eng.free(t)
        return y
    x = eng.random_dram(batch, hid, miburn.DRAW_NORMAL, 0.0, 1.0, base=1)
    gamma = eng.fill(1, hid, miburn.F32, 0x3F800000)
    wqkv, wo, wgu, wdn = bf((H + 2 * KVH) * D, hid, 2), bf(hid, H * D, 3), bf(2 * inter, hid, 4), bf(hid, inter, 5)
    cos = eng.random_dram(maxc, D, miburn.DRAW_UNIFORM, -1.0, 1.0, base=6)
    sin = eng.random_dram(maxc, D, miburn.DRAW_UNIFORM, -1.0, 1.0, base=7)
    kc = eng.random_dram(batch * KVH * maxc, D, miburn.DRAW_NORMAL, 0.0, 1.0, base=8)
    vc = eng.random_dram(batch * KVH * maxc, D, miburn.DRAW_NORMAL, 0.0, 1.0, base=9)
    span = (ctx + 1 + 63) // 64 * 64

    def layer():
        x1 = eng.norm_qkv_attention_o(x, gamma, 1e-5, wqkv, cos, sin, H, KVH, 0, ctx, span, kc, vc, D ** -0.5, wo)
        h = eng.norm_matvec(x1, gamma, 1e-5, wgu, 0, True)
        x2 = eng.norm_matvec(h, 0, 0.0, wdn, x1, False)
        for t in (x1, h, x2):
            eng.free(t)
    for _ in range(20):
        layer()
    eng.sync()
    eng.event_record(0)
    for _ in range(steps):
        layer()
    eng.event_record(1)
    eng.sync()
    us = eng.event_elapsed_ms(0, 1) * 1e3 / steps
    for t in (x, gamma, wqkv, wo, wgu, wdn, cos, sin, kc, vc):
        eng.free(t)
    return dict(batch=batch, ctx=ctx, steps=steps, us_per_layer=round(us, 2))


def prefill_bench(eng, batch: int = 1, prompt: int = 512, numerics: str = "reference", reps: int = 3) -> dict:
    """The SmolLM2-135M-shaped decoder's prefill alone (config 5's 512-token
    prompt, last-position logits), `reps` times after one warm run: a short
    run of few dispatches, for kernel traces and counters of the prefill's
    kernels (the whole decoder harness under rocprofv3 --pmc has ended in a
    fault inside the profiler)."""
    import miburn
    m = miburn.Llama(eng, miburn.SMOLLM2_135M, max_ctx=prompt, max_batch=batch, seed=5, numerics=numerics)
    ids = np.random.default_rng(9).integers(0, 49152, (batch, prompt)).astype(np.int32)

    def once():
        m.reset()
        eng.free(m.forward(ids))
    once()
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        once()
    eng.sync()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    m.close()
    return dict(batch=batch, prompt=prompt, numerics=numerics, reps=reps, prefill_ms=round(ms, 3))


def mlp_bench(eng, steps: int = 100, traces: bool = True) -> dict:
    """MLP 784->128->10 training, batch 64, SGD lr 0.01:
    eager steps on device-drawn batches, and the step captured as a trace
    replayed on host batches."""
    import miburn
    m = miburn.Mlp(eng)
    m.train_synthetic(64, 5, 0.01, data_seed=2)
    losses, ms = m.train_synthetic(64, steps, 0.01, data_seed=3)
    m.close()
    out = {"steps": steps, "ms_per_step": round(ms / steps, 4), "first_loss": round(float(losses[0]), 5),
           "last_loss": round(float(losses[-1]), 5)}
    if not traces:
        return out
    rng = np.random.default_rng(4)
    batches = [(rng.random((64, 784), dtype=np.float32), rng.integers(0, 10, (64, 1)).astype(np.int32))
               for _ in range(steps)]
    mt = miburn.Mlp(eng)
    x, lab = eng.upload(batches[0][0]), eng.upload_i32(batches[0][1])
    traced, replay = traced_steps(eng, lambda: mt.train_step_ids(x, lab, 0.01), (x, lab), batches)
    mt.close()
    eng.free(x)
    eng.free(lab)
    out.update(traced_ms_per_step=round(traced, 4), trace_replay_ms=round(replay, 4))
    return out


def transformer_bench(eng, steps: int = 20, traces: bool = True) -> dict:
    """4 layers, d_model 256, 4 heads, FFN 1024 GELU,
    LayerNorm, vocab 8192, seq 128, batch 16, fp32; uniform random tokens and
    targets; forward, cross-entropy, backward and SGD each step."""
    import miburn
    cfg = miburn.TRANSFORMER_CONFIG4
    B, S = 16, 128
    R, d, F, V, H = B * S, cfg["d_model"], cfg["d_ff"], cfg["vocab"], cfg["heads"]
    fwd = cfg["layers"] * (4 * 2 * R * d * d + 2 * 2 * R * d * F + 2 * 2 * B * H * S * S * (d // H)) + 2 * R * d * V
    m = miburn.Transformer(eng, cfg, seed=0)
    m.train_synthetic(B, S, 2, 0.05, data_seed=1)  # warm the kernels and the allocator
    losses, ms = m.train_synthetic(B, S, steps, 0.05, data_seed=2)
    m.close()
    step_ms = ms / steps
    out = {"steps": steps, "batch": B, "seq": S, "ms_per_step": round(step_ms, 3), "flop_per_step": 3 * fwd,
           "tflops": round(3 * fwd / (step_ms * 1e-3) / 1e12, 2),
           "first_loss": round(float(losses[0]), 4), "last_loss": round(float(losses[-1]), 4)}
    if not traces:
        return out
    rng = np.random.default_rng(5)
    batches = [tuple(rng.integers(0, V, (B * S, 1)).astype(np.int32) for _ in range(2)) for _ in range(steps)]
    mt = miburn.Transformer(eng, cfg, seed=0)
    tok, tgt = eng.upload_i32(batches[0][0]), eng.upload_i32(batches[0][1])
    traced, replay = traced_steps(eng, lambda: mt.train_step_ids(tok, tgt, B, S, 0.05), (tok, tgt), batches)
    mt.close()
    eng.free(tok)
    eng.free(tgt)
    out.update(traced_ms_per_step=round(traced, 3), trace_replay_ms=round(replay, 3))
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--dtype", choices=["bf16", "f32"], default="bf16")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--suite", action="store_true")
    ap.add_argument("--no-models", action="store_true")
    ap.add_argument("--only", choices=["decoder", "decode_layer", "prefill", "mlp", "transformer"],
                    help="run one model harness (or one decoder layer's decode launches) alone, for profiling, "
                         "and print its JSON")
    ap.add_argument("--batch", type=int, default=1, help="decoder batch for --only decoder / decode_layer")
    ap.add_argument("--numerics", choices=["reference", "performance"], default="reference",
                    help="decoder numeric contract for --only decoder")
    ap.add_argument("--no-traces", action="store_true",
                    help="skip the traced (HIP-graph) training and decode steps (under rocprofv3's kernel trace "
                         "graph replays are not followed, and a decode replay has ended in a host segfault)")
    ap.add_argument("--matmul-mode", choices=["fast", "accurate"], default=None,
                    help="how products with an F32 operand run (default: the engine's)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by output columns or rows with RCCL; nothing multi-GPU is built)",
              file=sys.stderr)
        return 2
    if args.suite:
        return suite(args.steps, args.matmul_mode)

    import miburn
    eng = miburn.Engine(0)
    if args.matmul_mode:
        eng.set_matmul_mode(miburn.MATMUL_FAST if args.matmul_mode == "fast" else miburn.MATMUL_ACCURATE)
    if args.only:
        out = {"decoder": lambda: decoder_bench(eng, args.batch, numerics=args.numerics, traced=not args.no_traces),
               "decode_layer": lambda: decode_layer_bench(eng, args.batch),
               "prefill": lambda: prefill_bench(eng, args.batch, numerics=args.numerics),
               "mlp": lambda: mlp_bench(eng, traces=not args.no_traces),
               "transformer": lambda: transformer_bench(eng, traces=not args.no_traces)}[args.only]()
        print(json.dumps({"harness": args.only, **out}), flush=True)
        eng.close()
        return 0
    n = args.n
    draw = miburn.DRAW_NORMAL
    a32 = eng.random_dram(n, n, draw, 0.0, 1.0, base=11)
    b32 = eng.random_dram(n, n, draw, 0.0, 1.0, base=12)
    if args.dtype == "bf16":
        a = eng.cast_float(a32, miburn.BF16)
        b = eng.cast_float(b32, miburn.BF16)
        eng.free(a32)
        eng.free(b32)
    else:
        a, b = a32, b32
    eng.sync()

    # Untimed warm-up: the W steps asked for, and at least WARM_S seconds of
    # the same product -- MI355X raises its clocks over a second or two of
    # sustained load (4096^3: ~1000-1080 TF/s in the first steps from idle,
    # ~1180 at steady state), and the timed steps measure the steady state.
    t_warm = time.perf_counter()
    done = 0
    while done < args.warmup or time.perf_counter() - t_warm < WARM_S:
        for _ in range(10):
            eng.free(eng.matmul_dram(a, False, b, False))
        done += 10
        eng.sync()

    eng.event_record(0)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        c = eng.matmul_dram(a, False, b, False)
        eng.free(c)
    eng.event_record(1)
    eng.sync()
    wall = time.perf_counter() - t0
    kernel_ms = eng.event_elapsed_ms(0, 1) / args.steps

    flop = 2.0 * n ** 3
    value = flop * args.steps / wall / 1e12
    achieved = flop / (kernel_ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[args.dtype]
    elt = 2 if args.dtype == "bf16" else 4
    traffic_min = (2 * n * n * elt + n * n * 4)
    line = {
        "metric": "matmul TFLOP/s (% MFMA peak) + SmolLM2-135M-shape decoder tokens/sec, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (device N(0,1) draws)",
        "config": {"workload": f"matmul {args.dtype}-in/f32-acc C=A.B {n}^3, A and B row-major (NN)",
                   "m": n, "n": n, "k": n},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": GEMM_TRAFFIC_BYTES.get((args.dtype, n)),
                     "kernel_ms": round(kernel_ms, 5), "min_hbm_bytes": traffic_min},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    if not args.no_models:
        line["decoder"] = [decoder_bench(eng, 1), decoder_bench(eng, 32)]
        line["decoder_performance_numerics"] = [decoder_bench(eng, 1, numerics="performance"),
                                                decoder_bench(eng, 32, numerics="performance")]
        line["mlp_train"] = mlp_bench(eng, traces=not args.no_traces)
        line["transformer_train"] = transformer_bench(eng, traces=not args.no_traces)
        if not args.no_cpu:
            cm = cpu_models_baseline()
            line["decoder"][0]["cpu_baseline"] = cm["decoder_b1"]
            line["decoder"][1]["cpu_baseline"] = cm["decoder_b32"]
            line["mlp_train"]["cpu_baseline"] = cm["mlp_train"]
            line["transformer_train"]["cpu_baseline"] = cm["transformer_train"]
    print(json.dumps(line), flush=True)
    eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
