"""Batch-1 greedy decode throughput of the hip device on the Qwen3-0.6B shape.

Workload: Qwen3-0.6B architecture (28 layers, hidden 1024, 16 Q / 8 KV heads,
head_dim 128, MLP 3072, vocab 151936, tied embeddings, q/k-norm, RoPE theta
1e6) with seeded synthetic N(0, 0.02) bf16 weights and RMSNorm gains of 1; a
16-token uniform-random prompt, then greedy decode. A step is one decode token
(one forward pass of one token through the whole model, on the device, plus the
greedy pick). The timed region holds exactly `--steps` decode steps from
position 16, after `--warmup` untimed steps; weights, caches and the prompt's
keys and values are resident in HBM before it starts.

Prints one JSON line (the benchmark contract) with the roofline of the decode
step and the CPU oracle's throughput on the same workload. Inside the same
line, `long_context_4b` reports the Qwen3-4B-shaped workload at the
reference's precision: an 8192-token prompt in f32 KV caches, then 256 greedy
decode steps (with its own roofline, the 8192-token prefill on the matrix
cores, and the CPU oracle at that context).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published


def kv_bytes_per_token(c, ctx_from: int, steps: int, kv_elem: int) -> float:
    """Average KV-cache bytes a decode step reads (every cached position, both
    caches, every layer) and writes (its own position)."""
    kvd = c.num_key_value_heads * c.head_dim()
    avg_ctx = sum(ctx_from + i + 1 for i in range(steps)) / steps
    read = c.num_hidden_layers * 2 * avg_ctx * kvd * kv_elem
    write = c.num_hidden_layers * 2 * kvd * kv_elem
    return read + write


def cpu_model_name() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads() -> tuple[int, int]:
    """(threads the CPU baseline uses, logical cores this process may run on):
    every core of the affinity mask, as rayon's default takes every logical
    core, unless OMP_NUM_THREADS sets the host's CPU share lower."""
    visible = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(visible, int(share)) if share.isdigit() and int(share) > 0 else visible
    return threads, visible


def cpu_baseline(cfg, weights, prompt, steps: int, repeats: int) -> dict:
    """The CPU oracle (C restatement of the reference's Cpu device and forward
    pass) on the same weights and prompt: greedy decode tokens/s from position
    len(prompt), median of `repeats` runs."""
    from oracle import ref

    cores, visible = cpu_threads()
    ref.set_threads(cores)
    model = ref.RefModel(cfg, weights)
    rates, tokens = [], []
    for _ in range(repeats):
        st = model.state(len(prompt) + steps)
        logits = model.forward(st, prompt, 0)
        toks = []
        t0 = time.perf_counter()
        for i in range(steps):
            tok = ref.argmax(logits)
            toks.append(tok)
            logits = model.forward(st, [tok], len(prompt) + i)
        rates.append(steps / (time.perf_counter() - t0))
        tokens = toks
    rates.sort()
    return {
        "value": rates[len(rates) // 2],
        "unit": "tokens/s",
        "cores": cores,
        "cores_visible": visible,
        "cpu": cpu_model_name(),
        "kind": "port",
        "sample": f"{steps} greedy decode steps after the {len(prompt)}-token prompt, median of {repeats} runs",
        "tokens": tokens,
    }


def cpu_baseline_at_context(cfg, weights, ctx: int, steps: int, first_token: int) -> dict:
    """The CPU oracle's greedy decode tokens/s at positions ctx, ctx + 1, ...
    over f32 caches holding ctx earlier positions. A prefill of ctx tokens is
    out of reach on the CPU, so the caches' earlier rows are filled with
    seeded N(0, 1) values instead (the oracle's time does not depend on
    them; rows left as untouched zero pages would read faster than real
    ones). One untimed step first, then `steps` timed ones."""
    from oracle import ref

    cores, visible = cpu_threads()
    ref.set_threads(cores)
    model = ref.RefModel(cfg, weights)
    st = model.state(ctx + steps + 1)
    kvd = cfg.num_key_value_heads * cfg.head_dim()
    rng = np.random.default_rng(ctx)
    rows = rng.standard_normal((ctx, kvd)).astype(np.float32)
    for layer in range(cfg.num_hidden_layers):
        for get in (ref.lib().ref_state_k_cache, ref.lib().ref_state_v_cache):
            cache = np.ctypeslib.as_array(ctypes.cast(get(st.handle, layer), ctypes.POINTER(ctypes.c_float)),
                                          shape=(st.max_len, kvd))
            cache[:ctx] = rows
    tok = int(first_token)
    logits = model.forward(st, [tok], ctx)
    t0 = time.perf_counter()
    for i in range(steps):
        tok = ref.argmax(logits)
        logits = model.forward(st, [tok], ctx + 1 + i)
    rate = steps / (time.perf_counter() - t0)
    del st
    return {
        "value": rate,
        "unit": "tokens/s",
        "cores": cores,
        "cores_visible": visible,
        "cpu": cpu_model_name(),
        "kind": "port",
        "sample": f"{steps} greedy decode steps at positions {ctx + 1}-{ctx + steps} over f32 caches of {ctx} "
                  "earlier positions (seeded values in place of a prefill), after one untimed step",
    }


def trait_path_decode(model, cfg, prompt, steps: int, paths: dict) -> dict:
    """Greedy decode through the Device-trait paths, as `titania run --device
    hip` would drive them: the prompt, then per step one forward of the
    picked token with its logits read back and the argmax taken on the host
    (model/chat.rs:149-178 at temperature 0 over Model::forward). OPS is the
    reference's unpatched forward_batch (one trait primitive per call), TRAIT
    the patched one (titania_amd/rust/patches: the fused trait-extension
    methods). Wall-clock tokens/s over `steps` steps after 4 untimed ones."""
    from titania_amd.model import State

    out = {}
    for name, path in paths.items():
        st = State(model, len(prompt) + steps + 4)
        logits = model.forward(st, prompt, 0, path)
        toks = []
        pos = len(prompt)
        for i in range(steps + 4):
            if i == 4:
                t0 = time.perf_counter()
            tok = int(np.argmax(logits))
            toks.append(tok)
            logits = model.forward(st, [tok], pos, path)
            pos += 1
        wall = time.perf_counter() - t0
        st.close()
        out[name] = {"value": steps / wall, "unit": "tokens/s", "ms_per_step": wall * 1000.0 / steps,
                     "tokens": toks}
    return out


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published


def prefill_flops(c, n: int) -> float:
    """Algorithmic flops of a forward over n prompt tokens from position 0:
    the layer GEMMs (2 n rows cols each), causal attention (scores and
    weighted values over n(n+1)/2 pairs per head) and the last token's lm_head."""
    H, I, hd = c.hidden_size, c.intermediate_size, c.head_dim()
    qd, kvd = c.num_attention_heads * hd, c.num_key_value_heads * hd
    gemm = 2.0 * n * (H * qd + 2 * H * kvd + qd * H + 3 * H * I)
    attn = 2.0 * 2.0 * hd * c.num_attention_heads * n * (n + 1) / 2
    return c.num_hidden_layers * (gemm + attn) + 2.0 * H * c.vocab_size


def prefill_bench(dev, model, cfg, n: int, kv: int, seed: int) -> dict:
    """A prompt of n uniform-random tokens through the fused forward (MFMA
    GEMMs for the projections), timed with HIP events on the device stream;
    median of 3 runs after one warmup."""
    from titania_amd import TH_PATH_FUSED, synth
    from titania_amd.model import State

    prompt = synth.prompt(n, cfg.vocab_size, seed=seed + 1)
    st = State(model, n, kv)
    model.forward(st, prompt, 0, TH_PATH_FUSED, want_logits=False)
    times = []
    for _ in range(3):
        dev.synchronize()
        dev.timer_begin()
        model.forward(st, prompt, 0, TH_PATH_FUSED, want_logits=False)
        times.append(dev.timer_end())
    st.close()
    ms = sorted(times)[1]
    fl = prefill_flops(cfg, n)
    return {"tokens": n, "ms": ms, "tokens_per_s": n / (ms / 1000.0),
            "roofline": {"bound": "mfma", "achieved": fl / (ms / 1000.0) / 1e12, "peak": MFMA_BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": fl / (ms / 1000.0) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                         "flops": fl}}


# Isolated decode kernels at the Qwen3-0.6B shapes: (name, rows, cols) of each
# GEMV, out = W x with W bf16 [rows, cols] and x f32 [cols].
KERNEL_GEMVS = [("q 1024->2048", 2048, 1024), ("k or v 1024->1024", 1024, 1024), ("o 2048->1024", 1024, 2048),
                ("gate+up 1024->6144", 6144, 1024), ("down 3072->1024", 1024, 3072),
                ("lm_head 1024->151936", 151936, 1024)]
KERNEL_CONTEXTS = [512, 4096, 32768]
ROTATE_BYTES = 1 << 30  # operand copies cycled per timed graph: well past the 256 MB last-level cache


def _graph_time(dev, calls, reps: int = 3, graph: bool = True) -> float:
    """Milliseconds of one replay of a graph holding `calls` (a list of
    zero-argument device calls), the median of `reps` timed replays after
    one untimed replay; without `graph`, of the calls launched one by one
    (the host's launch rate then bounds short kernels)."""
    if not graph:
        for c in calls:
            c()
        dev.synchronize()
        times = []
        for _ in range(reps):
            dev.timer_begin()
            for c in calls:
                c()
            times.append(dev.timer_end())
        return sorted(times)[len(times) // 2]
    dev.graph_begin()
    try:
        for c in calls:
            c()
    finally:
        g = dev.graph_end()
    g.launch()
    dev.synchronize()
    times = []
    for _ in range(reps):
        dev.timer_begin()
        g.launch()
        times.append(dev.timer_end())
    g.free()
    return sorted(times)[len(times) // 2]


def kernel_bench(dev, seed: int, graph: bool = True) -> dict:
    """Decode kernels alone: the GEMVs, RMSNorm and RoPE at the Qwen3-0.6B
    shapes (bf16 W and f32 x ~ N(0, 1)), and GQA decode attention (16 q heads,
    8 KV heads, head_dim 128) at contexts 512, 4096 and 32768 on the C ABI's
    f32 caches holding bf16-rounded N(0, 1). Each call is captured many times
    into one HIP graph over rotating copies of its operands (together past the
    last-level cache, so every call reads HBM), and a replay is timed with HIP
    events: the time per call includes the graph's gap between kernels
    (about 1.5 us). GB/s counts the algorithmic bytes of a call."""
    from titania_amd import Tensor
    from titania_amd.synth import bf16_to_f32, normal_bf16

    out = {"gemv": [], "norm_rope": [], "attention_f32_cache": []}
    rng = np.random.default_rng(seed)
    for name, rows, cols in KERNEL_GEMVS:
        wbits = normal_bf16(rows * cols, seed + rows + cols, name)
        copies = max(2, -(-ROTATE_BYTES // (2 * rows * cols)))
        ws = [dev.upload(Tensor((rows, cols), wbits)) for _ in range(copies)]
        x = dev.alloc(cols)
        dev.write(x, rng.standard_normal(cols).astype(np.float32))
        y = dev.alloc(rows)
        calls = [(lambda w=w: dev.matmul(y, w, x)) for w in ws] * max(1, 64 // copies)
        ms = _graph_time(dev, calls, graph=graph)
        us = ms * 1000.0 / len(calls)
        nbytes = 2 * rows * cols + 4 * cols + 4 * rows
        out["gemv"].append({"kernel": name, "us": us, "bytes": nbytes, "GB/s": nbytes / us / 1e3,
                            "frac": nbytes / us / 1e3 / HBM_PEAK_GBS, "copies": copies})
        for w in ws:
            w.free()
        x.free()
        y.free()
    gain = dev.upload(Tensor((1024,), normal_bf16(1024, seed, "gain")))
    hgain = dev.upload(Tensor((128,), normal_bf16(128, seed, "hgain")))
    xr = dev.alloc(1024)
    xh = dev.alloc(24 * 128)
    inv = (1e6 ** (-np.arange(64, dtype=np.float64) * 2.0 / 128)).astype(np.float32)
    ang = np.arange(4096, dtype=np.float32)[:, None] * inv[None, :]
    table = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32).reshape(-1)  # [pos][64][cos, sin]
    tb = dev.alloc(table.size)
    dev.write(tb, table)
    for name, call in [("rmsnorm 1 x 1024", lambda: dev.rmsnorm(xr, gain, 1e-6)),
                       ("rmsnorm 24 x 128 (q/k heads)", lambda: dev.rmsnorm(xh, hgain, 1e-6)),
                       ("rope 16 + 8 heads x 128", lambda: dev.rope(xh, tb, 4000, 24, 128))]:
        ms = _graph_time(dev, [call] * 64, graph=graph)
        out["norm_rope"].append({"kernel": name, "us": ms * 1000.0 / 64})
    for b in (gain, hgain):
        b.free()
    for b in (xr, xh, tb):
        b.free()
    H, KVH, hd = 16, 8, 128
    for ctx in KERNEL_CONTEXTS:
        n = ctx * KVH * hd
        kv_bytes = 2 * 4 * n
        copies = max(2, -(-ROTATE_BYTES // kv_bytes))
        kh = bf16_to_f32(normal_bf16(n, ctx, "k"))
        vh = bf16_to_f32(normal_bf16(n, ctx, "v"))
        ks, vs = [dev.alloc(n) for _ in range(copies)], [dev.alloc(n) for _ in range(copies)]
        for k, v in zip(ks, vs):
            dev.write(k, kh)
            dev.write(v, vh)
        q = dev.alloc(H * hd)
        dev.write(q, bf16_to_f32(normal_bf16(H * hd, ctx, "q")))
        o = dev.alloc(H * hd)
        dev.attention(o, q, ks[0], vs[0], ctx - 1, H, hd, KVH)  # sizes the device scratch before the capture
        calls = [(lambda k=k, v=v: dev.attention(o, q, k, v, ctx - 1, H, hd, KVH))
                 for k, v in zip(ks, vs)] * max(1, 32 // copies)
        ms = _graph_time(dev, calls, graph=graph)
        us = ms * 1000.0 / len(calls)
        nbytes = kv_bytes + 2 * 4 * H * hd
        out["attention_f32_cache"].append({"context": ctx, "us": us, "bytes": nbytes, "GB/s": nbytes / us / 1e3,
                                           "frac": nbytes / us / 1e3 / HBM_PEAK_GBS, "copies": copies})
        for b in ks + vs + [q, o]:
            b.free()
    return out


def long_context_decode(dev, model, cfg, kv: int, kv_elem: int, steps: int, seed: int) -> list:
    """Greedy decode of the whole model (one graph replay a step) after prompts
    of 512, 4096 and 32768 tokens, the product path's decode attention on the
    state's cache: ms per step and the step's algorithmic HBM rate (weights,
    the KV rows read and written, the logits)."""
    from titania_amd import TH_PATH_FUSED, synth
    from titania_amd.model import State

    rows = []
    for ctx in KERNEL_CONTEXTS:
        prompt = synth.prompt(ctx, cfg.vocab_size, seed=seed + ctx)
        st = State(model, ctx + steps + 1, kv)
        model.forward(st, prompt, 0, TH_PATH_FUSED, want_logits=False)
        model.decode(st, ctx, 2)  # captures the step graph
        model.forward(st, prompt, 0, TH_PATH_FUSED, want_logits=False)
        dev.synchronize()
        dev.timer_begin()
        model.decode(st, ctx, steps)
        ms = dev.timer_end() / steps
        st.close()
        nbytes = cfg.weight_bytes_per_token() + kv_bytes_per_token(cfg, ctx, steps, kv_elem) + 4 * cfg.vocab_size
        rows.append({"context": ctx, "ms_per_step": ms, "tokens_per_s": 1000.0 / ms, "bytes_per_step": nbytes,
                     "GB/s": nbytes / ms / 1e6, "frac": nbytes / ms / 1e6 / HBM_PEAK_GBS})
    return rows


LONG_CONTEXT = 8192


def long_context_4b(dev, seed: int, steps: int, warmup: int, cpu_steps: int) -> dict:
    """The Qwen3-4B-shaped workload (36 layers, hidden 2560, 32 Q / 8 KV heads,
    MLP 9728, vocab 151936, tied embeddings) at the reference's precision, f32
    KV caches: an 8192-token uniform-random prompt prefilled into the caches,
    then `steps` greedy decode steps, timed with HIP events on the device
    stream (weights, caches and the prompt's keys and values resident before
    the timed region). Also the 8192-token prefill alone on the matrix cores,
    and the CPU oracle's decode rate at the same context (bounded sample)."""
    from titania_amd import QWEN3_4B, TH_KV_F32, TH_PATH_FUSED, synth
    from titania_amd.model import Model, State

    cfg, ctx = QWEN3_4B, LONG_CONTEXT
    weights = synth.weights(cfg, seed=seed)
    prompt = synth.prompt(ctx, cfg.vocab_size, seed=seed + 2)
    model = Model(dev, cfg, weights)
    state = State(model, ctx + max(steps, warmup, 1), TH_KV_F32)
    model.forward(state, prompt, 0, TH_PATH_FUSED, want_logits=False)
    if warmup:
        model.decode(state, ctx, warmup)
    model.forward(state, prompt, 0, TH_PATH_FUSED, want_logits=False)
    dev.synchronize()
    dev.timer_begin()
    t0 = time.perf_counter()
    tokens = model.decode(state, ctx, steps)
    wall = time.perf_counter() - t0
    gpu_ms = dev.timer_end()
    state.close()
    nbytes = cfg.weight_bytes_per_token() + kv_bytes_per_token(cfg, ctx, steps, 4) + 4 * cfg.vocab_size
    achieved = nbytes / (gpu_ms / 1000.0 / steps) / 1e9
    traffic, traffic_source = measured_traffic("qwen3-4b", "f32", ctx)
    out = {
        "metric": "batch-1 decode tokens/s (Qwen3-4B shape, 8192-token prompt in the KV cache)",
        "value": steps / wall,
        "unit": "tokens/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": wall * 1000.0 / steps,
        "dtype": "bf16 weights; f32 activations, accumulation and KV cache",
        "config": {"workload": f"qwen3-4b greedy decode after an {ctx}-token prompt, {steps} steps, batch 1, "
                               "f32 KV cache", "model": "qwen3-4b", "prompt": ctx, "seq_len": ctx + steps},
        "roofline": {"bound": "hbm", "kernel": "decode step (one token's kernels; HIP graphs of eight steps "
                                               "replayed)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic, "traffic_source": traffic_source, "bytes_per_step": nbytes,
                     "gpu_ms_per_step": gpu_ms / steps},
        "prefill": prefill_bench(dev, model, cfg, ctx, TH_KV_F32, seed),
    }
    model.close()
    if cpu_steps:
        out["cpu_baseline"] = cpu_baseline_at_context(cfg, weights, ctx, cpu_steps, int(tokens[-1]))
    return out


TRAFFIC_FILE = ROOT / "profiles" / "decode_traffic.json"


def measured_traffic(model: str, kv: str, prompt: int):
    """HBM bytes per decode step (read + write) measured with hardware
    counters for this workload (model, KV cache type, prompt length), and
    where they come from (the commands, the source revision and the launch
    mode of that measurement), if a measurement is on file; else (None, None)."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None, None
    entry = data.get(f"{model}/{kv}/{prompt}")
    if entry is None:
        return None, None
    source = {k: entry[k] for k in ("revision", "mode", "commands") if k in entry}
    source["file"] = str(TRAFFIC_FILE.relative_to(ROOT))
    return entry.get("traffic_bytes_per_step"), source


def _counter_rows(directory: str):
    import csv

    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    with open(files[-1], newline="") as f:
        return list(csv.DictReader(f))


def pmc_summary(fetch_dir: str, write_dir: str, steps: int, copy_mib: int) -> dict:
    """Per-step HBM bytes from FETCH_SIZE and WRITE_SIZE (KiB per dispatch):
    the dispatches after the calibration copy are the timed decode steps; each
    counter is scaled by copy bytes / what it read for the copy."""
    if copy_mib <= 0:
        raise SystemExit("--pmc-summary needs --calibrate-copy MIB (the size the runs used)")
    copy_bytes = copy_mib * (1 << 20)
    out = {"steps": steps, "copy_bytes": copy_bytes}
    total = 0.0
    for name, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = [r for r in _counter_rows(directory) if r["Counter_Name"] == name]
        per_dispatch = {}
        kernel = {}
        for r in rows:
            d = int(r["Dispatch_Id"])
            per_dispatch[d] = per_dispatch.get(d, 0.0) + float(r["Counter_Value"])
            kernel[d] = r["Kernel_Name"]
        copies = [d for d in per_dispatch if "copy_kernel" in kernel[d]]
        if not copies:
            raise SystemExit(f"{name}: no copy_kernel dispatch in {directory}")
        c = max(copies)
        copy_kib = per_dispatch[c]
        after = sum(v for d, v in per_dispatch.items() if d > c)
        scale = (copy_bytes / 1024.0) / copy_kib
        step_bytes = after / steps * 1024.0 * scale
        out[name] = {"copy_kib": copy_kib, "scale": scale, "kib_per_step_raw": after / steps,
                     "bytes_per_step": step_bytes, "dispatches": sum(1 for d in per_dispatch if d > c)}
        total += step_bytes
    out["traffic_bytes_per_step"] = total
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=32, help="untimed decode steps before the timed ones")
    ap.add_argument("--prompt", type=int, default=16)
    ap.add_argument("--max-len", type=int, default=0,
                    help="positions the state's caches hold (0: prompt + steps, the default workload)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--kv", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--model", choices=["qwen3-0.6b", "qwen3-4b"], default="qwen3-0.6b")
    ap.add_argument("--prefill", type=int, default=512,
                    help="also time a prefill of this many random prompt tokens (0: skip)")
    ap.add_argument("--long-steps", type=int, default=256,
                    help="greedy decode steps of the Qwen3-4B-shaped workload after an 8192-token prompt with f32 "
                         "KV caches, reported inside the line as long_context_4b (0: skip it)")
    ap.add_argument("--long-cpu-steps", type=int, default=4,
                    help="CPU-oracle decode steps timed at that context")
    ap.add_argument("--trait-steps", type=int, default=32,
                    help="also time greedy decode through the Device-trait paths (ops, trait) for this many steps "
                         "(0: skip)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--cpu-repeats", type=int, default=3)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="before the timed steps, copy a MIB-MiB buffer once with the library's copy kernel: a "
                         "known-size reference for the hardware byte counters (see --pmc-summary)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="instead of benchmarking, summarize two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "'bench.py --calibrate-copy MIB --steps K' into HBM bytes per decode step")
    ap.add_argument("--kernels", action="store_true",
                    help="instead of the decode benchmark, time the decode kernels alone (GEMVs, norms, RoPE, "
                         "attention at contexts 512 / 4096 / 32768) and whole-model decode after prompts of those "
                         "lengths; prints one JSON line")
    ap.add_argument("--no-graph", action="store_true",
                    help="with --kernels, launch the calls one by one instead of replaying them in HIP graphs")
    args = ap.parse_args()

    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, steps=args.steps, copy_mib=args.calibrate_copy)))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the decode path runs on a single MI355X and --gpus {args.gpus} "
              "is not supported (no multi-GPU sharding is built).", file=sys.stderr)
        return 2

    from titania_amd import (QWEN3_0_6B, QWEN3_4B, TH_KV_BF16, TH_KV_F32, TH_PATH_FUSED, TH_PATH_OPS, TH_PATH_TRAIT,
                             Hip, synth)
    from titania_amd.model import Model, State

    cfg = QWEN3_0_6B if args.model == "qwen3-0.6b" else QWEN3_4B
    kv = TH_KV_F32 if args.kv == "f32" else TH_KV_BF16
    kv_elem = 4 if kv == TH_KV_F32 else 2

    if args.kernels:
        dev = Hip(0)
        res = {"mode": "kernels", "data": "synthetic (seeded N(0,1) operands; model weights N(0,0.02))",
               "peak_GB/s": HBM_PEAK_GBS, "graphs": not args.no_graph,
               "isolated": kernel_bench(dev, args.seed, graph=not args.no_graph)}
        print(json.dumps(res["isolated"]), file=sys.stderr, flush=True)
        model = Model(dev, cfg, synth.weights(cfg, seed=args.seed))
        res["decode_after_prompt"] = {"model": args.model, "kv": args.kv, "steps": args.steps,
                                      "rows": long_context_decode(dev, model, cfg, kv, kv_elem, args.steps, args.seed)}
        print(json.dumps(res))
        return 0

    t = time.perf_counter()
    weights = synth.weights(cfg, seed=args.seed)
    prompt = synth.prompt(args.prompt, cfg.vocab_size, seed=args.seed)
    gen_s = time.perf_counter() - t

    dev = Hip(0)
    model = Model(dev, cfg, weights)
    K, W = args.steps, args.warmup
    state = State(model, max(args.max_len, args.prompt + max(K, W, 1)), kv)

    # Warmup: prefill, W decode steps (captures the decode graph).
    model.forward(state, prompt, 0, TH_PATH_FUSED, want_logits=False)
    if W:
        model.decode(state, args.prompt, W)
    # Timed: the prompt is re-run first (rewriting positions 0..15), then exactly K steps.
    model.forward(state, prompt, 0, TH_PATH_FUSED, want_logits=False)
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        a, b = dev.alloc(n), dev.alloc(n)
        dev.copy(b, 0, a, 0, n)
        dev.synchronize()
        a.free()
        b.free()
    dev.synchronize()
    dev.timer_begin()
    t0 = time.perf_counter()
    tokens = model.decode(state, args.prompt, K)
    wall = time.perf_counter() - t0
    gpu_ms = dev.timer_end()
    ms_per_step = wall * 1000.0 / K

    weight_bytes = cfg.weight_bytes_per_token()
    kvb = kv_bytes_per_token(cfg, args.prompt, K, kv_elem)
    logits_bytes = 4 * cfg.vocab_size
    bytes_per_token = weight_bytes + kvb + logits_bytes
    achieved = bytes_per_token / (gpu_ms / 1000.0 / K) / 1e9
    mode = os.environ.get("TITANIA_DECODE", "graph")
    kernel = {
        "eager": "decode step (one token's kernels launched one by one)",
    }.get(mode, "decode step (one token's kernels; HIP graphs of eight steps replayed)")
    traffic, traffic_source = (None, None) if args.max_len else measured_traffic(args.model, args.kv, args.prompt)

    out = {
        "metric": "batch-1 decode tokens/s (Qwen3-0.6B shape) + % of HBM GB/s roofline",
        "value": K / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"bf16 weights; f32 activations, accumulation and {args.kv} KV cache",
        "data": "synthetic (seeded N(0,0.02) bf16 weights, gains 1, uniform-random prompt)",
        "config": {
            "workload": f"{args.model} greedy decode, {args.prompt}-token prompt, {K} steps, batch 1, "
                        f"{args.kv} KV cache" + (f" of {args.max_len} positions" if args.max_len else ""),
            "model": args.model,
            "global_batch": 1,
            "seq_len": args.prompt + K,
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source": traffic_source,
            "bytes_per_step": bytes_per_token,
            "gpu_ms_per_step": gpu_ms / K,
        },
        "synth_s": gen_s,
    }
    if args.prefill:
        out["prefill"] = prefill_bench(dev, model, cfg, args.prefill, kv, args.seed)
    if args.trait_steps and kv == TH_KV_F32:
        tp = trait_path_decode(model, cfg, prompt, args.trait_steps, {"ops": TH_PATH_OPS, "trait": TH_PATH_TRAIT})
        fused = [int(x) for x in tokens]
        for v in tp.values():
            n = min(len(fused), len(v["tokens"]))
            v["tokens_match_fused"] = v.pop("tokens")[:n] == fused[:n]
        tp["note"] = ("side figures, not the metric: the Device-trait paths with the logits read and the argmax "
                      "taken on the host every step; ops = the reference's forward_batch over the hip device's "
                      "primitives, trait = the patched forward_batch over its fused trait methods")
        out["trait_paths"] = tp
    if not args.no_cpu:
        cb = cpu_baseline(cfg, weights, prompt, K, args.cpu_repeats)
        out["parity_tokens_match"] = [int(x) for x in tokens] == cb.pop("tokens")
        out["cpu_baseline"] = cb
    state.close()
    model.close()
    if args.long_steps:
        del weights
        out["long_context_4b"] = long_context_4b(dev, args.seed, args.long_steps, 8,
                                                 0 if args.no_cpu else args.long_cpu_steps)
    print(json.dumps(out))
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
