#!/usr/bin/env python3
"""Headline benchmark: batch-1 greedy decode tok/s of a Qwen2.5-0.5B-shaped model
with int4-g128 layer weights and an int8 output head,
on one MI355X through libqwen_hip.so.

A step is one decode token: one replay of the hipGraph-captured decode step
(24 layers -> lm_head -> argmax -> next token, all on the device; each step's argmax and
the next token's gather are made by the next step's first launch, and a decode call ends
with one pick launch of its own). The
KV cache is first filled from a seeded 1024-token prompt (untimed); W warmup
steps run and are rewound; then exactly K steps are timed with HIP events on the
library's stream (and wall clock around them), inputs resident in HBM.

Also reported on the same JSON line:
  roofline       the dominant kernel of the step (the most in-situ time per token),
                 algorithmic bytes per launch over its back-to-back launch duration, vs
                 8 TB/s; the same figures for every role under "roles"
  per_kernel_us  in-situ microseconds per token by kernel role (events around
                 every launch, the reference's decode-profile split), and each role's
                 launch duration back to back
  decode_bounds  what bounds the step on this device: the pure streaming-read ceiling, and
                 the cost of a graph-replayed launch that reads its predecessor's output (as
                 every decode launch does) times the step's launches
  decode_kernels_cold  the step's own launches (int4 qkv / o / gate-up / down, int8 head,
                 split-K attention) each over copies of its operands past 512 MiB, GB/s and
                 the fraction of 8 TB/s and of the read ceiling
  matvec_isolated  BASELINE config 2: int8 matvec with an f16 activation at the
                 five layer shapes, one list-driven launch over >= 512 MiB of
                 distinct matrices (larger than the 256 MB last-level cache)
  attention_decode  BASELINE config 3: split-K GQA attention over f16 caches at contexts
                 128 .. 32768, one list-driven launch over >= 512 MiB of distinct caches
  prefill_512    BASELINE config 5: time to first token of a 512-token prompt through each
                 matmul path (per-position matvec, 8-position batched tiles, MFMA)
  loader         the load path's conversion kernels (bf16 checkpoint -> int8 / int4 / f16
                 on the device) in GB/s, and the whole model load, host- vs device-converted
  path_comparison  the same-session comparison of the matmul paths (web/scaling.html): the
                 paths checked to compute the same model, then prompt time-to-logits at 1 ..
                 512 tokens and single-token steps, median/min/max per path
  perplexity     the reference's perplexity protocol on a seeded 48-token passage (no tokenizer
                 or checkpoint here): f16 / int8 / int4-g128 / int4-g32 scored one token at a time
                 on the decode kernels, paired NLL change vs f16 +- SE, and |dNLL| vs the oracle
  greedy_match   every timed token against the CPU oracle continuing from the GPU's cache
                 (teacher-forced), the smallest top-2 margin, and per layer the max-abs
                 relative error and cosine of the K/V rows the decoded positions stored
  cpu_baseline   the reference's src/cpu path restated in JavaScript (oracle/cpu_model.js)
                 timed under Node on one host core over a bounded sample of the same
                 workload; cpu_baseline_c the C oracle on the same sample

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 16]
"""
import argparse
import json
import os
import re
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llm-inference-webgpu_amd"))

import qwen_hip as H  # noqa: E402

PEAK_HBM_GBS = 8000.0
PROBE_AFTER = 64  # the roofline probe's row: this many positions past the prompt (at most the timed steps)
LOGIT_REL = 1e-4        # test/model.test.js:40; web/scaling.html:122-127 holds its non-bitwise path to it
METRIC = "batch-1 decode tok/s, Qwen2.5-0.5B int4/int8; matvec HBM GB/s vs peak"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def role_bytes(cfg, ctx_len, group=128):
    """Algorithmic HBM bytes per launch of each decode role (int4-g128 layers, int8
    head, f16 cache): weights + their scales/zeros once, plus the activations each
    launch must read and write."""
    d, kv, ffn, V = cfg.hidden, cfg.kv_dim, cfg.intermediate, cfg.vocab

    def int4(rows, cols):
        return rows * cols // 2 + rows * (cols // group) * 8

    f = 4
    return {
        "embed": d * 2 + d * f,
        "qkv": int4(d + 2 * kv, d) + (d + 2 * kv) * f + 2 * d * f + (d + 2 * kv) * f,
        "attention": 2 * ctx_len * kv * 2 + (d + 2 * kv) * f + 2 * kv * 2 + d * f,
        "oproj": int4(d, d) + d * f + 2 * d * f,
        "gateup": int4(2 * ffn, d) + 2 * d * f + ffn * f,
        "down": int4(d, ffn) + ffn * f + 2 * d * f,
        "head": V * d + V * f + 2 * d * f + V * f,
    }


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_int4_ctx1024_hbm_traffic.md")


def measured_traffic(role, context):
    """HBM bytes per launch of a decode role from the committed rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes (each scaled by a 64 MiB copy kernel's reading), taken at context 1024;
    None for another context or without the profile."""
    if context != 1024:
        return None
    try:
        with open(TRAFFIC_PROFILE) as f:
            m = re.search(r"```json\n(.*?)\n```", f.read(), re.S)
        return json.loads(m.group(1))["bytes_per_launch"].get(role) if m else None
    except (OSError, ValueError, KeyError):
        return None


def isolated_matvec(ctx, shapes, reps=5):
    """Config 2: weights W ~ N(0, 0.02) quantized per row to int8 by the reference quantizer's
    rule (the device quantizer, qh_quantize), x ~ N(0,1) f16, one list-driven launch over
    >= 512 MiB of distinct matrices (copies of the quantized matrix at distinct addresses)."""
    out = {}
    rng = np.random.default_rng(2)
    for name, rows, cols in shapes:
        per = rows * cols + 4 * rows                   # codes + scales stored
        count = int(np.ceil((512 << 20) / per))
        algo = rows * cols + 4 * rows + 2 * cols + 4 * rows   # + x read + y written
        w = ctx.upload((rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)))
        dq, ds = ctx.empty(count * rows * cols, np.int8), ctx.empty(count * rows * 4)
        ctx.quantize(w, H.FMT_F32, rows, cols, H.FMT_INT8, data=dq, scales=ds)
        w.free()
        for z in range(1, count):
            ctx.copy(dq, 0, dq, z * rows * cols, rows * cols)
            ctx.copy(ds, 0, ds, z * rows * 4, rows * 4)
        x = rng.standard_normal(cols).astype(np.float16).view(np.uint16)
        dx, dy = ctx.upload(x), ctx.empty(count * rows * 4)
        W = ctx.weight(H.FMT_INT8, rows, cols, dq, ds)
        ctx.matvec_xh_list(W, count, rows * cols, rows, dx, 0, dy)   # warm
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for _ in range(reps):
            ctx.matvec_xh_list(W, count, rows * cols, rows, dx, 0, dy)
        ctx.record(e1)
        ms = ctx.elapsed_ms(e0, e1) / reps
        ctx.destroy_event(e0), ctx.destroy_event(e1)
        gbs = count * algo / (ms * 1e-3) / 1e9
        out[name] = {"shape": [rows, cols], "matrices": count, "bytes_per_launch": count * algo,
                     "us_per_launch": round(ms * 1e3, 2), "us_per_matrix": round(ms * 1e3 / count, 4),
                     "GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"isolated int8 matvec {name} {rows}x{cols} x{count}: {gbs:.0f} GB/s")
        for b in (dq, ds, dx, dy):
            b.free()
    return out


def decode_bounds(ctx, launches_per_step, graphs=True):
    """What bounds the batch-1 decode step on this device: the pure streaming-read ceiling
    (1 GiB), and the cost of a graph-replayed launch of 224 blocks that does nothing, reads
    nothing it depends on, or reads the vector the previous launch wrote (as each decode launch
    reads its predecessor's output) -- times the step's latency floor. graphs=False (the
    --launch direct runs made for profilers that do not follow graph launches) leaves the
    launch probes out."""
    ceiling = ctx.read_ceiling(1 << 30, 10)
    if not graphs:
        return {"read_ceiling_GBps": round(ceiling, 1), "read_ceiling_frac": round(ceiling / PEAK_HBM_GBS, 4),
                "launch_us": None, "step_launches": launches_per_step, "step_floor_us": None}
    empty = ctx.launch_floor(0)
    static = ctx.launch_floor(2)
    dependent = ctx.launch_floor(1)
    out = {"read_ceiling_GBps": round(ceiling, 1), "read_ceiling_frac": round(ceiling / PEAK_HBM_GBS, 4),
           "launch_us": {"empty": round(empty, 3), "no_dependency": round(static, 3),
                         "reads_previous_output": round(dependent, 3)},
           "step_launches": launches_per_step,
           "step_floor_us": round(launches_per_step * dependent, 1)}
    log(f"bounds: read ceiling {ceiling:.0f} GB/s; launch {empty:.2f} us empty, {dependent:.2f} us dependent; "
        f"step floor {out['step_floor_us']} us over {launches_per_step} launches")
    return out


def cold_decode_kernels(model, cache, cfg, ctx_len, ceiling, reps=5):
    """The decode step's own launches timed cold: one launch over copies of the role's operands
    exceeding 512 MiB (qh_decode_kernel_time_cold). Bytes per copy are what streams from HBM:
    the weights with their scales and zero points (int4-g128 layers, int8 head), or for the
    attention the f16 K and V chunks of 64 positions its slots read at position ctx_len."""
    d, kv, ffn, V = cfg.hidden, cfg.kv_dim, cfg.intermediate, cfg.vocab
    int4 = lambda r, c: r * c // 2 + r * (c // 128) * 8
    per_copy = {"qkv": int4(d + 2 * kv, d), "oproj": int4(d, d), "gateup": int4(2 * ffn, d),
                "down": int4(d, ffn), "head": V * d + 4 * V,
                "attention": ((ctx_len + 1 + 63) // 64) * 64 * kv * 2 * 2}
    out = {}
    cache.length = ctx_len
    for role in ("qkv", "attention", "oproj", "gateup", "down", "head"):
        us, copies = model.kernel_time_cold(cache, role, 512 << 20, reps)
        nbytes = copies * per_copy[role]
        gbs = nbytes / (us * 1e-6) / 1e9
        out[role] = {"copies": copies, "bytes_per_launch": nbytes, "us_per_launch": round(us, 2),
                     "GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
        if ceiling:
            out[role]["frac_of_read_ceiling"] = round(gbs / ceiling, 4)
        log(f"cold {role}: {copies} copies, {us:.1f} us, {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%} of 8 TB/s)")
    return out


class _Ptr:
    """A device address inside a larger DeviceBuffer (what the operator bindings take)."""

    def __init__(self, ptr):
        self.ptr = ptr


def stream_decode_kernels(model, cache, cfg, ctx_len, ceiling, reps=5, totals=(512, 1024, 2048)):
    """The decode step's matrix kernels over the same >= 512 MiB of operand copies as
    cold_decode_kernels, on a grid sized for streaming instead of for one step's latency
    (qh_decode_kernel_time_stream); each block stages its activation once and walks many rows
    with the next rows' loads in flight. down and the head: blocks_per_copy blocks per copy, so
    that the launch has about `total` blocks (the best total is reported). qkv, o-proj and
    gate|up run as a flat list, whose grid the library sizes to the device's resident blocks
    (blocks_per_copy does not change it). The library checks each list launch's outputs bit for
    bit against the step's own launch shape."""
    d, kv, ffn, V = cfg.hidden, cfg.kv_dim, cfg.intermediate, cfg.vocab
    int4 = lambda r, c: r * c // 2 + r * (c // 128) * 8
    per_copy = {"qkv": int4(d + 2 * kv, d), "oproj": int4(d, d), "gateup": int4(2 * ffn, d),
                "down": int4(d, ffn), "head": V * d + 4 * V}
    out = {}
    cache.length = ctx_len
    for role in ("qkv", "oproj", "gateup", "down", "head"):
        best = None
        for total in totals:
            copies = int(np.ceil((512 << 20) / per_copy[role]))
            bpc = max(1, int(round(total / copies)))
            us, copies = model.kernel_time_stream(cache, role, bpc, 512 << 20, reps)
            gbs = copies * per_copy[role] / (us * 1e-6) / 1e9
            if best is None or gbs > best["GBps"]:
                best = {"blocks_per_copy": bpc, "copies": copies,
                        "bytes_per_launch": copies * per_copy[role], "us_per_launch": round(us, 2),
                        "GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
        if ceiling:
            best["frac_of_read_ceiling"] = round(best["GBps"] / ceiling, 4)
        out[role] = best
        log(f"stream {role}: {best['blocks_per_copy']} blocks per copy, {best['GBps']:.0f} GB/s "
            f"({best['frac']:.1%} of 8 TB/s)")
    return out


def attention_sweep(ctx, contexts=(128, 1024, 4096, 32768), heads=14, kv_heads=2, reps=5):
    """Config 3: one query (position ctx-1) against f16 K/V caches of N(0,1) values, through the
    list form of the split-K operator: one launch over a rotation of distinct caches totalling
    >= 512 MiB (larger than the last-level cache). Algorithmic bytes per cache: K and V (512 B
    per position over both kv heads) + q read + out written."""
    out = {}
    rng = np.random.default_rng(3)
    for n_ctx in contexts:
        cap = n_ctx
        vstride = H.value_cache_bytes(cap, kv_heads) // (kv_heads * 64 * 2)
        k_elems, v_elems = kv_heads * cap * 64, kv_heads * 64 * vstride
        per = k_elems + v_elems
        copies = int(np.ceil((512 << 20) / (2 * per)))
        block = rng.standard_normal(min(per, 1 << 22)).astype(np.float16)
        buf = ctx.upload(np.tile(block, int(np.ceil(copies * per / block.size)))[:copies * per])
        q = ctx.upload(rng.standard_normal(heads * 64).astype(np.float32))
        o = ctx.empty(copies * heads * 64 * 4)
        algo = 2 * 2 * kv_heads * 64 * n_ctx + 2 * heads * 64 * 4
        kc, vc = _Ptr(buf.ptr), _Ptr(buf.ptr + 2 * k_elems)
        ctx.attention_list(q, kc, vc, per, per, copies, cap, o, n_ctx - 1, heads, kv_heads)   # warm
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for _ in range(reps):
            ctx.attention_list(q, kc, vc, per, per, copies, cap, o, n_ctx - 1, heads, kv_heads)
        ctx.record(e1)
        ms = ctx.elapsed_ms(e0, e1) / reps
        ctx.destroy_event(e0), ctx.destroy_event(e1)
        gbs = copies * algo / (ms * 1e-3) / 1e9
        out[str(n_ctx)] = {"caches": copies, "bytes_per_launch": copies * algo,
                           "us_per_launch": round(ms * 1e3, 2), "us_per_cache": round(ms * 1e3 / copies, 4),
                           "GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"attention ctx {n_ctx} x{copies}: {gbs:.0f} GB/s, {ms * 1e3 / copies:.3f} us per cache")
        for b in (buf, q, o):
            b.free()
    return out


def prefill_bench(ctx, cfg, ckpt, seed, prompt_len=512, modes=("matvec", "batched", "mfma")):
    """Config 5: time-to-first-token of a seeded prompt with int8 layers and head, through
    one decode step per position, the reference's 8-position tiles, and the MFMA contraction.
    A token's time is wall clock around forward(): the ids' upload, the embedding gather, all
    layers, the head and the logits readback; best of 3. `ttft_ms` replays the prompt shape's
    graph (captured on the shape's second use, before the timed runs), `ttft_ms_direct` launches
    every kernel from the host."""
    model = H.GpuModel.load_checkpoint(ctx, ckpt, cfg, "int8", 128, "int8", maxPositions=prompt_len + 8)
    prompt = H.synth_tokens(seed, "config5.prompt", cfg.vocab, prompt_len)
    res = {}
    logits = {}
    def best_of(cache, n=3):
        best = r = None
        for _ in range(n):
            cache.length = 0
            t0 = time.perf_counter()
            r = model.forward_tokens(prompt, cache)
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return best, r

    for mode in modes:
        model.set_matmul(mode)
        cache = model.newCache(prompt_len + 8)
        model.forward_tokens(prompt, cache)   # warm (allocations, code objects)
        model.decode_use_graph(cache, False)  # every kernel launched directly
        direct, _ = best_of(cache)
        model.decode_use_graph(cache, True)   # the shape's second use captures its graph
        cache.length = 0
        model.forward_tokens(prompt, cache)
        best, r = best_of(cache)              # replays
        logits[mode] = r
        res[mode] = {"ttft_ms": round(best * 1e3, 2), "prompt_tok_per_s": round(prompt_len / best, 1),
                     "ttft_ms_direct": round(direct * 1e3, 2)}
        cache.destroy()
        log(f"prefill {prompt_len} ({mode}): {best * 1e3:.2f} ms replayed, {direct * 1e3:.2f} ms launched directly")
    if "batched" not in logits:
        model.destroy()
        return res
    ref = logits["batched"]["logits"].astype(np.float64)
    for mode in [m for m in ("matvec", "mfma") if m in logits]:
        got = logits[mode]["logits"].astype(np.float64)
        res[mode]["logits_rel_vs_batched"] = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
        res[mode]["argmax_equal"] = logits[mode]["argmax"] == logits["batched"]["argmax"]
    lin = 2 * prompt_len * sum(r * c for r, c in (
        (cfg.hidden + 2 * cfg.kv_dim, cfg.hidden), (cfg.hidden, cfg.hidden),
        (2 * cfg.intermediate, cfg.hidden), (cfg.hidden, cfg.intermediate))) * cfg.layers
    res["linear_gflop"] = round(lin / 1e9, 1)
    if "mfma" in res:
        res["mfma_linear_tflops_lower_bound"] = round(lin / (res["mfma"]["ttft_ms"] * 1e-3) / 1e12, 1)
    model.destroy()
    return res


def perplexity_bench(ctx, cfg, ckpt, seed, n=48, oracle_check=True):
    """The reference's perplexity protocol (web/perplexity.html:125-215, validate/perplexity.js)
    on a seeded n-token passage of this synthetic model -- no tokenizer or checkpoint is here:
    every scheme scores the same n - 1 positions one token at a time through the cache
    (qh_score: the decode kernels reading the int8/int4 codes), perplexity = exp(mean NLL), and
    the paired per-position NLL change against f16 with its standard error (the reference's
    "not distinguishable" test at 2 SE). Layers and head use the scheme, as the reference's
    round trip covers the tied embedding; input rows are the bf16 rows. With the oracle check,
    the C oracle scores the same positions on the same quantized weights: the largest |dNLL|
    is the device arithmetic's own effect."""
    ids = H.synth_tokens(seed, "perplexity.passage", cfg.vocab, n)
    if oracle_check:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as O
        O.lib().or_set_threads(host_cpu()[1])
    schemes = [("f16", "f16", 128, 16.0), ("int8", "int8", 128, 8 + 32 / cfg.hidden),
               ("int4-g128", "int4", 128, 4 + 64 / 128), ("int4-g32", "int4", 32, 4 + 64 / 32)]
    rows, base = {}, None
    for label, scheme, group, bits in schemes:
        model = H.GpuModel.load_checkpoint(ctx, ckpt, cfg, scheme, group, scheme, maxPositions=n + 8)
        cache = model.newCache(n + 2)
        t0 = time.perf_counter()
        nll = model.score(ids, cache)
        dt = time.perf_counter() - t0
        cache.destroy()
        model.destroy()
        row = {"bits_per_weight": round(bits, 3), "perplexity": round(float(np.exp(nll.mean())), 4),
               "mean_nll": round(float(nll.mean()), 6), "scored": int(nll.size), "seconds": round(dt, 3)}
        if base is None:
            base = nll
        else:
            d = nll - base
            se = float(np.std(d, ddof=1) / np.sqrt(d.size))
            row["paired_mean_nll_delta_vs_f16"] = round(float(d.mean()), 6)
            row["paired_standard_error"] = round(se, 6)
            row["distinguishable_at_2se"] = bool(abs(d.mean()) >= 2 * se)
        if oracle_check:
            oracle = O.OracleModel(cfg, ckpt, scheme=scheme, group=group, lm_head=scheme, kv_f16=True)
            oc = oracle.new_cache(n + 2)
            ref = np.array([O.nll(oracle.forward([ids[t]], oc), ids[t + 1]) for t in range(n - 1)])
            row["oracle_perplexity"] = round(float(np.exp(ref.mean())), 4)
            row["max_abs_nll_vs_oracle"] = float(f"{np.max(np.abs(nll - ref)):.3g}")
        rows[label] = row
        log(f"perplexity {label}: {row['perplexity']} over {row['scored']} positions"
            + (f", |dNLL| vs oracle <= {row['max_abs_nll_vs_oracle']}" if oracle_check else ""))
    return {"protocol": f"seeded {n}-token passage, full left context, one token at a time, nothing scored twice, "
                        f"{n - 1} positions", "schemes": rows}


def host_cpu():
    """The host CPU's model name and the threads this process may use (the box's share)."""
    name = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return name, min(usable or 1, int(os.environ.get("OMP_NUM_THREADS", "16")))


def node_version():
    try:
        return subprocess.run(["node", "--version"], capture_output=True, text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None


def node_cpu_baseline(cfg, ckpt, cache, first, gpu_tokens, steps, context):
    """The reference CPU path in JavaScript (oracle/cpu_model.js: src/cpu/model.js restated for
    Node 12, f32 storage, f64 sums) timed under Node on one thread: the int4-g128 layers and int8
    head from the reference quantizer's arrays, dequantized once at load, the KV cache holding
    the GPU run's context (the same f16 values), then `steps` greedy decode steps. Returns the
    baseline record and the token match, or (None, None) without Node."""
    version = node_version()
    if version is None:
        log("cpu baseline: node not found; skipped")
        return None, None
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    bits = O.js_cache_bits([cache.present(L) for L in range(cfg.layers)], context)
    with tempfile.TemporaryDirectory() as d:
        manifest = O.write_js_manifest(d, cfg, ckpt, scheme="int4", group=128, kv_f16=True, cache_bits=bits,
                                       context=context, first=first, steps=steps)
        res = O.run_js_model(manifest, timeout=900)
    toks = res["tokens"]
    compared = min(len(toks), len(gpu_tokens))
    match = sum(int(a == b) for a, b in zip(toks[:compared], gpu_tokens[:compared]))
    cpu_name, _ = host_cpu()
    cpu = {"value": round(steps / res["seconds"], 4), "unit": "tok/s", "cores": 1, "kind": "port",
           "sample": f"{steps} greedy decode steps at context {context}..{context + steps - 1} (KV cache "
                     f"loaded from the GPU run), oracle/cpu_model.js under Node {version}, 1 thread on "
                     f"{cpu_name} ({os.cpu_count()} CPUs visible); {res['perStepSeconds']:.2f} s per token"}
    return cpu, f"{match}/{compared}"


def greedy_check(cfg, ckpt, cache, first, gpu_tokens, context):
    """Every timed GPU token against the C oracle (the reference CPU path's arithmetic)
    continuing from the GPU's cache: teacher-forced, each step fed the GPU's previous token, so
    one disagreement would not hide the others (src/cpu/model.js:174-187). Runs on the threads
    the box gives this process. Returns matched/compared, the smallest top-2 logit margin
    and the time taken."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    _, threads = host_cpu()
    O.lib().or_set_threads(threads)
    oracle = O.OracleModel(cfg, ckpt, scheme="int4", group=128, lm_head="int8", kv_f16=True)
    oc = oracle.new_cache(context + len(gpu_tokens))
    oc.load_device(cache, context)
    fed = [first] + [int(t) for t in gpu_tokens[:-1]]
    matched, margins = 0, []
    t0 = time.perf_counter()
    for i, tok in enumerate(fed):
        logits = oracle.forward([tok], oc)
        matched += int(O.argmax(logits) == gpu_tokens[i])
        top = np.partition(logits.astype(np.float64), -2)[-2:]
        margins.append(float(top[1] - top[0]))
    seconds = time.perf_counter() - t0
    return {"matched_compared": f"{matched}/{len(fed)}", "min_top2_margin": round(min(margins), 6),
            "teacher_forced": True, "oracle": "oracle/liboracle.so (f64 sums)", "threads": threads,
            "seconds": round(seconds, 1), "per_layer": per_layer_kv(cfg, cache, oc, context, len(fed))}


def per_layer_kv(cfg, cache, oc, start, n):
    """Each layer's output at the decoded positions start..start+n-1 -- the K and V rows it
    stored -- on the GPU against the oracle's for the same fed tokens: max-abs relative (over
    max |oracle|) and cosine per layer (test/model.test.js:39 holds layers to 5e-4). Both
    caches hold f16 values; the oracle's were computed from its own f64 sums."""
    def rel(a, b):
        return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))

    def cos(a, b):
        return float(a.ravel() @ b.ravel() / (np.linalg.norm(a) * np.linalg.norm(b)))

    out = {"positions": [start, start + n - 1], "layers": cfg.layers}
    for kind in ("key", "value"):
        errs, coss = [], []
        for L in range(cfg.layers):
            a = cache.present(L)[kind][:, start:start + n].astype(np.float64)
            b = oc.present(L)[kind][:, start:start + n].astype(np.float64)
            errs.append(rel(a, b))
            coss.append(cos(a, b))
        out[f"{kind}_max_abs_rel"] = [float(f"{e:.3g}") for e in errs]
        out[f"{kind}_cosine"] = [round(c, 9) for c in coss]
    out["worst_max_abs_rel"] = max(max(out["key_max_abs_rel"]), max(out["value_max_abs_rel"]))
    out["min_cosine"] = min(min(out["key_cosine"]), min(out["value_cosine"]))
    return out


def cpu_baseline(cfg, ckpt, cache, first, gpu_tokens, steps, context):
    """The oracle (a C port of the reference CPU path, f64 accumulation) on one core:
    its KV cache is loaded with the GPU cache's context (the same f16 values), then it
    greedy-decodes `steps` tokens. Returns the baseline record and the token match."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    O.lib().or_set_threads(1)
    oracle = O.OracleModel(cfg, ckpt, scheme="int4", group=128, lm_head="int8", kv_f16=True)
    oc = oracle.new_cache(context + steps)
    oc.load_device(cache, context)
    toks, tok = [], first
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = O.argmax(oracle.forward([tok], oc))
        toks.append(tok)
    dt = time.perf_counter() - t0
    O.lib().or_set_threads(host_cpu()[1])
    compared = min(steps, len(gpu_tokens))
    match = sum(int(a == b) for a, b in zip(toks[:compared], gpu_tokens[:compared]))
    cpu = {"value": round(steps / dt, 4), "unit": "tok/s", "cores": 1, "kind": "port",
           "sample": f"{steps} greedy decode steps at context {context}..{context + steps - 1} "
                     f"(KV cache loaded from the GPU run), oracle/liboracle.so, 1 thread on "
                     f"{host_cpu()[0]} ({os.cpu_count()} CPUs visible)"}
    return cpu, f"{match}/{compared}"


def mfma_same_f16_check(model, cfg, ckpt, hidden, seq):
    """The MFMA path's logits for a prompt against the CPU oracle attending to that run's own f16
    cache rows (the same-input comparison of web/kernels.html:51-54): max-abs relative. Two paths
    with f16 caches are not compared with each other, because an entry that rounds to the
    neighbouring f16 value in one of them moves later positions in that one only."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    model.set_matmul("mfma")
    cache = model.newCache(seq + 2)
    got = model.forward(hidden, seq, cache)["logits"].astype(np.float64)
    oracle = O.OracleModel(cfg, ckpt, scheme="int8", lm_head="int8", kv_f16=True)
    oc = oracle.new_cache(seq + 2)
    oc.load_device(cache, seq, pin=True)
    oc.length = 0
    ref = oracle.forward_hidden(hidden, seq, oc).astype(np.float64)
    cache.destroy()
    return float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))


def scaling_bench(ctx, cfg, ckpt, lengths=(1, 8, 32, 52, 64, 128, 256, 512, 1024), repeats=5,
                  decode_steps=24, paths=("matvec", "batched", "mfma"), oracle_check=True):
    """The same-session path comparison of web/scaling.html:40-194: time-to-logits of a prompt
    through each matmul path (median/min/max of `repeats`, the path order rotated every repeat),
    after a check at 52 tokens that the paths compute the same model (batched bit-identical to
    matvec; MFMA with the same argmax and within the reference's 1e-4 of the CPU oracle on its own
    f16 cache rows, mfma_same_f16_check), then single-token forward steps after a
    32-token prompt, the paths alternating step by step on caches of their own. int8 layers and
    head (the MFMA path contracts int8/int4); the embedding rows come from the host as the page
    gathers them, so each timing is of the forward pass alone."""
    model = H.GpuModel.load_checkpoint(ctx, ckpt, cfg, "int8", 128, "int8", maxPositions=max(lengths) + 64)
    d = cfg.hidden
    longest = max(max(lengths), 32 + decode_steps) + 2
    emb = ckpt["model.embed_tokens.weight"]
    ids = (1000 + 7 * np.arange(longest)) % cfg.vocab                 # web/scaling.html:69
    hidden = H.bf16_to_f32(emb[ids]).reshape(-1)

    def prefill(path, seq):
        model.set_matmul(path)
        cache = model.newCache(seq + 2)
        t0 = time.perf_counter()
        out = model.forward(hidden[:seq * d], seq, cache)
        ms = (time.perf_counter() - t0) * 1e3
        cache.destroy()
        return ms, out

    for path in paths:                       # first use of every tile shape and code object
        for seq in (1, 2, 4, 8, 64):
            prefill(path, seq)
    outs = {p: prefill(p, 52)[1] for p in paths}
    m, b = outs["matvec"]["logits"], outs["batched"]["logits"]
    agree = {"logits": int(m.size), "batched_differing": int(np.sum(m.view(np.uint32) != b.view(np.uint32))),
             "argmax": {p: outs[p]["argmax"] for p in paths}}
    if "mfma" in outs:
        agree["mfma_max_relative"] = float(np.max(np.abs(outs["mfma"]["logits"].astype(np.float64) - m))
                                           / np.max(np.abs(m)))
        if oracle_check:
            agree["mfma_vs_same_f16_cpu"] = mfma_same_f16_check(model, cfg, ckpt, hidden[:52 * d], 52)
    ok = agree["batched_differing"] == 0 and len(set(agree["argmax"].values())) == 1 and \
        agree.get("mfma_vs_same_f16_cpu", 0.0) <= LOGIT_REL
    if not ok:
        raise RuntimeError(f"paths disagree: {json.dumps(agree)}")

    def summary(runs):
        return {"median": round(float(np.median(runs)), 3), "min": round(min(runs), 3), "max": round(max(runs), 3)}

    rows = []
    for seq in lengths:
        runs = {p: [] for p in paths}
        for i in range(repeats):
            for k in range(len(paths)):
                p = paths[(k + i) % len(paths)]
                runs[p].append(prefill(p, seq)[0])
        row = {"seq": seq, **{p: summary(runs[p]) for p in paths}}
        row["speedup_vs_matvec"] = {p: round(row["matvec"]["median"] / row[p]["median"], 2) for p in paths[1:]}
        rows.append(row)
        log(f"scaling prefill {seq}: " + ", ".join(f"{p} {row[p]['median']:.2f} ms" for p in paths))
    caches = {}
    for p in paths:
        model.set_matmul(p)
        caches[p] = model.newCache(32 + decode_steps + 2)
        model.forward(hidden[:32 * d], 32, caches[p])
    steps = {p: [] for p in paths}
    for i in range(decode_steps):
        row_x = hidden[(32 + i) * d:(33 + i) * d]
        for k in range(len(paths)):
            p = paths[(k + i) % len(paths)]
            model.set_matmul(p)
            t0 = time.perf_counter()
            model.forward(row_x, 1, caches[p])
            steps[p].append((time.perf_counter() - t0) * 1e3)
    for c in caches.values():
        c.destroy()
    model.destroy()
    decode = {p: {**summary(steps[p]), "tok_per_s": round(1e3 / float(np.median(steps[p])), 1)} for p in paths}
    log(f"scaling decode step: " + ", ".join(f"{p} {decode[p]['median']:.3f} ms" for p in paths))
    return {"agree": agree, "prefill": rows, "decode_after_32": decode, "repeats": repeats,
            "weights": "int8 layers, int8 head", "timing": "wall clock around forward(), logits read back"}


def loader_bench(ctx, cfg, ckpt, reps=10):
    """The loader's conversion kernels (qh_quantize) over bf16 checkpoint tensors resident in
    HBM -- the output projection and every layer's gate|up and down matrices, each set as one
    launch -- timed with HIP events on the library's stream over `reps` back-to-back launches;
    algorithmic bytes = the bf16 source read once + the codes, scales and zero points written.
    Then the whole model loaded both ways: host quantizer + upload, and device conversion."""
    d, V = cfg.hidden, cfg.vocab
    layers = range(cfg.layers)
    gate_up = np.concatenate([ckpt[f"model.layers.{i}.mlp.{p}_proj.weight"] for i in layers for p in ("gate", "up")])
    down = np.concatenate([ckpt[f"model.layers.{i}.mlp.down_proj.weight"] for i in layers])
    embed = ckpt["model.embed_tokens.weight"]
    cases = [("lm_head_int8", embed, H.FMT_INT8, 0), ("gate_up_int4", gate_up, H.FMT_INT4, 128),
             ("down_int4", down, H.FMT_INT4, 128), ("lm_head_f16", embed, H.FMT_F16, 0)]
    out = {}
    for label, bits, fmt, group in cases:
        rows, cols = bits.shape
        n = rows * cols
        src = ctx.upload(bits)
        data, scales, zeros = ctx.quantize(src, H.FMT_BF16, rows, cols, fmt, group)   # warm
        e0, e1 = ctx.event(), ctx.event()
        ctx.done()
        ctx.record(e0)
        for _ in range(reps):
            ctx.quantize(src, H.FMT_BF16, rows, cols, fmt, group, data, scales, zeros)
        ctx.record(e1)
        us = ctx.elapsed_ms(e0, e1) * 1e3 / reps
        ctx.destroy_event(e0), ctx.destroy_event(e1)
        written = {H.FMT_INT8: n + 4 * rows, H.FMT_INT4: n // 2 + 8 * (n // max(group, 1)), H.FMT_F16: 2 * n}[fmt]
        nbytes = 2 * n + written
        gbs = nbytes / (us * 1e-6) / 1e9
        out[label] = {"shape": [rows, cols], "us_per_launch": round(us, 1), "bytes_per_launch": nbytes,
                      "GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"convert {label} {rows}x{cols}: {us:.1f} us, {gbs:.0f} GB/s")
        for b in (src, data, scales, zeros):
            if b is not None:
                b.free()
    del gate_up, down
    t0 = time.perf_counter()
    tensors = H.device_tensors(ckpt, cfg, "int4", 128, "int8")
    model = H.GpuModel.load(ctx, tensors, cfg, maxPositions=64)
    host_s = time.perf_counter() - t0
    model.destroy()
    del tensors
    t0 = time.perf_counter()
    model = H.GpuModel.load_checkpoint(ctx, ckpt, cfg, "int4", 128, "int8", maxPositions=64)
    device_s = time.perf_counter() - t0
    model.destroy()
    out["model_load_s"] = {"host_quantize_then_upload": round(host_s, 2), "device_convert": round(device_s, 2),
                           "host_cpus": os.cpu_count()}
    log(f"model load: host quantizer {host_s:.2f} s, device conversion {device_s:.2f} s")
    return out


def copy_calibration(mib, reps=5):
    """qh_copy of `mib` MiB, `reps` times: per dispatch it reads and writes exactly mib MiB, the
    scale for the FETCH_SIZE / WRITE_SIZE counters."""
    ctx = H.GpuContext.create(0)
    n = mib << 20
    src, dst = ctx.empty(n, np.uint8), ctx.empty(n, np.uint8)
    ctx.copy(src, 0, dst, 0, n)
    ctx.done()
    for _ in range(reps):
        ctx.copy(src, 0, dst, 0, n)
    ctx.done()
    print(json.dumps({"copy_bytes": n, "launches": reps + 1, "kernel": "k_copy16"}), flush=True)
    src.free(), dst.free()
    ctx.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--context", type=int, default=1024)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-steps", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--isolated", choices=["all", "none"], default="all",
                    help="the isolated config-2 matvec, config-3 attention and config-5 prefill lines")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run qh_copy over this many MiB, 5 times: the known-size kernel that the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE passes are calibrated against")
    ap.add_argument("--prefill-only", choices=["all", "batched", "mfma"], default=None,
                    help="only the config-5 prefill (the named matmul modes), for profiling it alone")
    ap.add_argument("--scaling", action="store_true",
                    help="only the same-session comparison of the matmul paths over prompt lengths")
    ap.add_argument("--loader-only", action="store_true",
                    help="only the loader's conversion kernels and the two whole-model loads")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the config-3 attention list over contexts 128..32768 (for profiling it)")
    ap.add_argument("--perplexity-only", action="store_true",
                    help="only the perplexity protocol over the four weight schemes")
    ap.add_argument("--cold-only", action="store_true",
                    help="only the decode step's launches timed cold over >= 512 MiB of operand "
                         "copies after the prompt (step grids, then streaming grids), for the "
                         "rocprofv3 counter passes over them")
    ap.add_argument("--launch", choices=["graph", "direct"], default="graph",
                    help="decode by hipGraph replay (default) or direct launches of the same "
                         "kernels (for profilers that do not follow graph launches)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: batch-1 decode of a 0.5B model runs on a single GPU and "
              "is not sharded across several. Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_mib:
        copy_calibration(args.copy_mib)
        return

    cfg = H.QWEN25_05B
    ctx = H.GpuContext.create(0)
    log(ctx.describe())
    t0 = time.perf_counter()
    ckpt = H.synthesize_checkpoint(cfg, seed=args.seed)
    if args.prefill_only:
        modes = ("matvec", "batched", "mfma") if args.prefill_only == "all" else (args.prefill_only,)
        print(json.dumps({"prefill_512": prefill_bench(ctx, cfg, ckpt, args.seed, modes=modes)}), flush=True)
        ctx.close()
        return
    if args.loader_only:
        print(json.dumps({"loader": loader_bench(ctx, cfg, ckpt)}), flush=True)
        ctx.close()
        return
    if args.scaling:
        print(json.dumps({"scaling": scaling_bench(ctx, cfg, ckpt)}), flush=True)
        ctx.close()
        return
    if args.attention_only:
        print(json.dumps({"attention_decode": attention_sweep(ctx)}), flush=True)
        ctx.close()
        return
    if args.perplexity_only:
        print(json.dumps({"perplexity": perplexity_bench(ctx, cfg, ckpt, args.seed, oracle_check=not args.no_cpu)}),
              flush=True)
        ctx.close()
        return
    extra = max(args.steps, args.warmup, args.profile_steps, args.cpu_steps) + 1
    capacity = args.context + extra
    model = H.GpuModel.load_checkpoint(ctx, ckpt, cfg, "int4", 128, "int8", maxPositions=capacity)
    log(f"model ready in {time.perf_counter() - t0:.1f}s, {model.device_bytes / 1e6:.1f} MB on device")

    prompt = H.synth_tokens(args.seed, "config4.prompt", cfg.vocab, args.context)
    cache = model.newCache(capacity)
    model.decode_use_graph(cache, args.launch == "graph")
    t0 = time.perf_counter()
    first = model.forward_tokens(prompt, cache)["argmax"]
    prefill_s = time.perf_counter() - t0
    log(f"prefilled {args.context} positions in {prefill_s:.2f}s (8-position batched tiles)")

    if args.cold_only:
        print(json.dumps({"decode_kernels_cold": cold_decode_kernels(model, cache, cfg, args.context, None),
                          "decode_kernels_streaming": stream_decode_kernels(model, cache, cfg, args.context, None)}),
              flush=True)
        cache.destroy()
        model.destroy()
        ctx.close()
        return

    # The decode graphs are captured and uploaded here, outside the timed region.
    if args.launch == "graph":
        model.decode_prepare(cache)
    if args.warmup:
        model.decode(cache, first, args.warmup)
        cache.length = args.context

    e0, e1 = ctx.event(), ctx.event()
    ctx.done()
    w0 = time.perf_counter()
    ctx.record(e0)
    model.decode_launch(cache, first, args.steps)
    ctx.record(e1)
    tokens = model.decode_collect(cache, args.steps)
    wall = time.perf_counter() - w0
    ms = ctx.elapsed_ms(e0, e1)
    ctx.destroy_event(e0), ctx.destroy_event(e1)
    tok_s = args.steps / (ms / 1e3)
    log(f"decode: {args.steps} steps in {ms:.2f} ms (events), {wall * 1e3:.2f} ms (wall): {tok_s:.0f} tok/s")

    # Each role's own launches probed at a fixed row, the 65th after the prompt whatever the
    # number of timed tokens (so the line and the committed traces, taken over 64 steps, describe
    # the same launch; the rows the decode stored below it stay as decoded, since a role launch
    # appends K/V at its own position only): 240 of the step's launches of it back to back on the
    # library's stream between two events (no event between launches; its 24 weight sets
    # cache-resident), then one launch cold over >= 512 MiB of copies.
    probe = args.context + min(args.steps, PROBE_AFTER)
    cache.length = probe
    back_to_back = {r: round(model.kernel_time(cache, r, 240), 3)
                    for r in ("qkv", "attention", "oproj", "gateup", "down", "head")}
    cold = cold_decode_kernels(model, cache, cfg, probe, None)
    stream = stream_decode_kernels(model, cache, cfg, probe, None)

    # In-situ per-kernel times over the same positions.
    cache.length = args.context
    psteps = min(args.profile_steps, args.steps)
    ptoks, roles = model.decode_profile(cache, first, psteps)
    deterministic = bool(np.array_equal(ptoks, tokens[:psteps]))
    if psteps < args.steps:
        # The timed decode's later rows again (the same kernels on the same tokens), so the cache
        # holds every timed position for the oracle comparison below.
        rest = model.decode(cache, int(ptoks[-1]), args.steps - psteps)
        deterministic = deterministic and bool(np.array_equal(rest, tokens[psteps:]))
    rb = role_bytes(cfg, args.context + psteps // 2)
    per_kernel = {}
    for r, (tot_ms, n) in roles.items():
        if n == 0:
            continue
        per_kernel[r] = {"us_per_token": round(tot_ms * 1e3 / psteps, 2),
                         "us_per_launch": round(tot_ms * 1e3 / n, 3),
                         "launches_per_token": n // psteps,
                         "GBps": round(rb[r] * n / (tot_ms * 1e-3) / 1e9, 1)}
    for r in per_kernel:
        if r in back_to_back:
            per_kernel[r]["us_back_to_back"] = back_to_back[r]
    # Every role's roofline figure: algorithmic bytes per launch at the probe position over the
    # role's back-to-back launch duration (240 of the step's own launches between two events, so
    # no event sits between them; a kernel tracer's average over the same launches agrees within
    # ~10%). The dominant kernel is the role with the most in-situ time per token (the event split
    # above), which ranks the roles as a kernel trace of the step does; back-to-back durations of
    # the attention, gate/up and down lie within a few % of each other and would trade places
    # from run to run.
    pb = role_bytes(cfg, probe)
    roles_roof = {}
    for r in ("qkv", "attention", "oproj", "gateup", "down", "head"):
        if r not in per_kernel:
            continue
        us = back_to_back[r]
        gbs = pb[r] / (us * 1e-6) / 1e9
        roles_roof[r] = {"us_per_launch": us, "in_situ_us_per_token": per_kernel[r]["us_per_token"],
                         "bytes_per_launch": pb[r], "achieved": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
    dominant = max(roles_roof, key=lambda r: roles_roof[r]["in_situ_us_per_token"])
    d = roles_roof[dominant]
    roofline = {"bound": "hbm", "kernel": dominant, "achieved": d["achieved"],
                "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": d["frac"],
                "traffic": measured_traffic(dominant, args.context), "bytes_per_launch": d["bytes_per_launch"],
                "us_per_launch": d["us_per_launch"], "roles": roles_roof}
    log(f"per-kernel: {json.dumps(per_kernel)}")

    # What bounds the step; the cold launches against the read ceiling.
    bounds = decode_bounds(ctx, sum(v["launches_per_token"] for v in per_kernel.values()),
                           graphs=args.launch == "graph")
    for v in list(cold.values()) + list(stream.values()):
        v["frac_of_read_ceiling"] = round(v["GBps"] / bounds["read_ceiling_GBps"], 4)

    iso = attn = prefill = loader = paths = ppl = None
    if args.isolated == "all":
        d, kv, ffn, V = cfg.hidden, cfg.kv_dim, cfg.intermediate, cfg.vocab
        iso = isolated_matvec(ctx, [("q_o", d, d), ("k_v", kv, d), ("gate_up", ffn, d),
                                    ("down", d, ffn), ("lm_head", V, d)])
        attn = attention_sweep(ctx)
        prefill = prefill_bench(ctx, cfg, ckpt, args.seed)
        loader = loader_bench(ctx, cfg, ckpt)
        paths = scaling_bench(ctx, cfg, ckpt, lengths=(1, 8, 64, 256, 512), repeats=3, decode_steps=12,
                              oracle_check=not args.no_cpu)
        ppl = perplexity_bench(ctx, cfg, ckpt, args.seed, oracle_check=not args.no_cpu)

    cpu = match = cpu_c = match_c = greedy = None
    if not args.no_cpu:
        # Every timed token against the oracle first (all threads), then the 1-thread baselines.
        greedy = greedy_check(cfg, ckpt, cache, first, tokens, args.context)
        log(f"greedy tokens vs the CPU oracle: {greedy['matched_compared']} (teacher-forced), "
            f"min top-2 margin {greedy['min_top2_margin']}, {greedy['seconds']} s on {greedy['threads']} threads")
        # The reference CPU path under Node (the baseline), and the C oracle beside it.
        cpu, match = node_cpu_baseline(cfg, ckpt, cache, first, tokens, args.cpu_steps, args.context)
        if cpu:
            log(f"cpu baseline (node): {cpu['value']} tok/s, greedy match {match}")
        cpu_c, match_c = cpu_baseline(cfg, ckpt, cache, first, tokens, args.cpu_steps, args.context)
        log(f"cpu oracle (C): {cpu_c['value']} tok/s, greedy match {match_c}")
        if cpu is None:
            cpu, match = cpu_c, match_c

    line = {
        "metric": METRIC, "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int4",
        "data": "synthetic (seeded random-init weights, seeded prompt ids)",
        "config": {"workload": "config4: Qwen2.5-0.5B-shape int4-g128 decode, int8 lm_head, "
                               f"f16 KV cache, context {args.context}, batch 1, greedy",
                   "global_batch": 1, "seq_len": args.context, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_c": cpu_c,
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
        "per_kernel_us": per_kernel,
        "profile_tokens_match_timed": deterministic,
        "greedy_match": greedy,
        "greedy_match_cpu_sample": match,
        "greedy_match_cpu_c_sample": match_c,
        "decode_bounds": bounds,
        "decode_kernels_cold": cold,
        "decode_kernels_streaming": stream,
        "matvec_isolated": iso,
        "attention_decode": attn,
        "prefill_512": prefill,
        "loader": loader,
        "path_comparison": paths,
        "perplexity": ppl,
        "prefill_s": round(prefill_s, 3),
    }
    print(json.dumps(line), flush=True)
    cache.destroy()
    model.destroy()
    ctx.close()


if __name__ == "__main__":
    main()
