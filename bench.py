"""Benchmark of the MI355X sparse expert reader (one JSON line on stdout).

Workload (`--config`, default c2): the configuration the headline metric is
quoted on that fits one GPU -- a stack of L distinct synthetic MoE layers
(random-init BF16 weights, their ternary sketches and rank-32 recovery maps),
each with its own decode batch of T tokens routed by a softmax router. One
step replays a HIP graph holding the L reader calls on one stream; the reported
value is microseconds per layer (the median of the measurement plan's samples;
`ms_per_step` is the mean of exactly the timed steps).

Also reported: tokens/s, the algorithmic HBM bytes of each layer call (per
expert touched: union of kept coordinates' code runs, FP16 scale plane and FP32
norms, union of kept channels' gate/up and down rows, union of skipped
channels' encoder rows; plus U, signs, inputs and outputs), the achieved GB/s,
a live per-stage kernel timing whose dominant stage gives the roofline object,
and the CPU oracle on the C1 layer as the CPU baseline.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "calibration-free-moe_amd"), ROOT]

import numpy as np  # noqa: E402
import torch  # noqa: E402

from calibration_free_moe.reader import _ext  # noqa: E402
from calibration_free_moe.reader.budget import compile_budget  # noqa: E402
from calibration_free_moe.reader.progressive import (  # noqa: E402
    GROUPED_TOKENS,
    ProgressiveReader,
    ReaderWorkspace,
    channel_major_down,
)
from calibration_free_moe.reader.sketch import block_hadamard_signs, build_sketch  # noqa: E402
from calibration_free_moe.recovery import subspace_bank  # noqa: E402

METRIC = "sparse MoE-layer decode µs/layer at batch 1/64/128; achieved HBM GB/s on bytes read"
HBM_PEAK_GBPS = 8000.0

CONFIGS = {
    # name: (hidden, width, experts, top_k, layers, tokens, retention, keep, description)
    "c1": (2048, 1024, 64, 8, 1, 1, 0.123, 0.625, "OLMoE-1B-7B layer, batch 1"),
    "c2": (2048, 1024, 64, 8, 16, 64, 0.123, 0.625, "OLMoE-1B-7B layer x16, batch 64"),
    "c3": (2048, 768, 128, 8, 48, 1, 0.123, 0.625, "Qwen3-30B-A3B layer x48"),
    "c4": (2048, 768, 128, 8, 48, 256, 0.123, 0.625,
           "Qwen3-30B-A3B layer x48, Zipf(1.2) expert popularity"),
    "c5": (2048, 512, 256, 8, 16, 1, 0.123, 0.625,
           "256-expert I=512 layer x16, dense I=512 shared expert beside it"),
}
# c4 routes the c3 layers' weights with skewed popularity (same weight seeds)
WEIGHT_SEEDS = {"c1": 1, "c2": 2, "c3": 3, "c4": 3, "c5": 5}
ZIPF = {"c4": 1.2}
SHARED_WIDTH = {"c5": 512}


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def device_weights(hidden, width, experts, rank, seed, device, std=0.02):
    """One synthetic layer's weights, generated on the GPU (recipe of tests/synthetic.py)."""
    g = torch.Generator(device=device).manual_seed(seed)
    gate_up = (torch.randn(experts, 2 * width, hidden, generator=g, device=device) * std).bfloat16()
    down = (torch.randn(experts, hidden, width, generator=g, device=device) * std).bfloat16()
    router = (torch.randn(experts, hidden, generator=g, device=device) * std).bfloat16()
    u, b, _ = subspace_bank(down, rank)
    encoder = b.bfloat16()
    decoder = u.bfloat16().contiguous()
    codes, stats = build_sketch(gate_up, block_hadamard_signs(hidden, device))
    return {
        "gate_up": gate_up, "down": channel_major_down(down), "encoder": encoder,
        "decoder": decoder, "sketch": (codes, stats), "router": router,
    }


def device_inputs(weights, tokens, top_k, seed, device, zipf=None):
    """A routed decode batch: N(0, 1) states with 1 % of dims x20, softmax top-k.

    With `zipf` = s the experts are drawn instead with popularity p_e
    proportional to rank^-s (a seeded permutation of the experts): top-k
    without replacement by Gumbel-top-k on log p_e, weights the renormalised
    softmax of the chosen perturbed scores (recipe of tests/synthetic.py).
    """
    hidden = weights["router"].shape[1]
    experts = weights["router"].shape[0]
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(tokens, hidden, generator=g, device=device)
    dims = torch.randperm(hidden, generator=g, device=device)[: max(1, round(0.01 * hidden))]
    x[:, dims] *= 20
    x = x.bfloat16()
    if zipf is None:
        logits = (x.float() @ weights["router"].float().T).bfloat16().float()
        probabilities, ids = torch.softmax(logits, -1).topk(top_k, -1)
        probabilities = (probabilities / probabilities.sum(-1, keepdim=True)).float().contiguous()
    else:
        rank = torch.arange(1, experts + 1, dtype=torch.float64, device=device)
        popularity = rank.pow(-zipf)
        permutation = torch.randperm(experts, generator=g, device=device)
        log_p = torch.log(popularity / popularity.sum())[permutation]
        uniform = torch.rand(tokens, experts, generator=g, device=device, dtype=torch.float64)
        scores = log_p[None, :] - torch.log(-torch.log(uniform))
        ids = scores.topk(top_k, dim=-1).indices
        probabilities = torch.softmax(scores.gather(1, ids), dim=-1).float().contiguous()
    return {"hidden": x, "ids": ids.to(torch.int64).contiguous(), "weights": probabilities,
            "out": torch.empty_like(x)}


def device_layer(hidden, width, experts, top_k, rank, tokens, seed, device):
    data = device_weights(hidden, width, experts, rank, seed, device)
    data.update(device_inputs(data, tokens, top_k, seed + 7, device))
    return data


def algorithmic_bytes(reader: ProgressiveReader, tokens: int) -> dict[str, int]:
    """Bytes one call must read: per-expert unions over the batch (host count)."""
    p = reader.plan
    h, i, k = p.hidden_size, p.expert_width, p.top_k
    blocks = h // 128
    rank = reader.rank
    ids = reader.ids[:tokens].cpu().numpy()
    selected = reader.selected[:tokens].cpu().numpy().reshape(tokens, k, i).astype(bool)
    keep = p.screen_coordinates
    coords = (reader.sketch_coordinates[:tokens].cpu().numpy() if keep < 128
              else np.broadcast_to(np.arange(128), (tokens, blocks, 128)))
    run = 32 * -(-2 * ((i + 4) // 5) // 32)
    planes = 1 + (reader.selection_score != "point")
    totals = {"sketch": 0, "gate_up": 0, "down": 0, "encoder": 0, "fixed": 0}
    for expert in np.unique(ids):
        rows = np.argwhere(ids == expert)
        union_coords = 0
        for b in range(blocks):
            union_coords += len(np.unique(coords[rows[:, 0], b].reshape(-1)))
        totals["sketch"] += union_coords * run + blocks * 2 * i * 2 * planes + 4 * i
        kept = np.zeros(i, bool)
        skipped = np.zeros(i, bool)
        for t, slot in rows:
            kept |= selected[t, slot]
            skipped |= ~selected[t, slot]
        totals["gate_up"] += int(kept.sum()) * 4 * h
        totals["down"] += int(kept.sum()) * 2 * h
        totals["encoder"] += int(skipped.sum()) * 2 * rank
    totals["fixed"] = 2 * h * rank + h + tokens * (2 * h + 2 * h + 8 * k)
    totals["total"] = sum(totals.values())
    return totals


STAGE_BYTES = {"screen": ("sketch",), "exact": ("gate_up",), "down": ("down",),
               "encode": ("encoder",)}
DIRECT_RANK = 32  # rank at which the encoder runs inside the exact launch
STAGE_KERNELS = {"prepare": "prepare_kernel", "screen": "small_screen_kernel",
                 "select": "select_kernel", "exact": "exact_kernel",
                 "encode": "encode_kernel", "down": "down_kernel", "output": "output_kernel"}
GROUP_EXACT_TOKENS = GROUPED_TOKENS  # batches from which the exact stage runs group_exact_kernel
WIDE_OUTPUT_TOKENS = 64  # batches from which the output stage runs output_wide_kernel (top-k <= 16)


def encoder_in_exact(tokens: int, rank: int) -> bool:
    """Whether the exact launch also runs the recovery encoder (the encode
    stage then launches nothing)."""
    return rank == DIRECT_RANK


def stage_bytes(stage: str, tokens: int, rank: int) -> tuple[str, ...]:
    """Algorithmic byte groups read by a stage's launch."""
    if encoder_in_exact(tokens, rank):
        if stage == "exact":
            return ("gate_up", "encoder")
        if stage == "encode":
            return ()
    return STAGE_BYTES.get(stage, ())


def stage_kernel(stage: str, tokens: int) -> str:
    """Name of the kernel a stage launches at this batch size (the screen
    launch also scores; the score stage launches nothing)."""
    if stage == "exact" and tokens >= GROUP_EXACT_TOKENS:
        return "group_exact_kernel"
    if stage == "screen" and tokens >= _ext.FUSED_SCREEN_TOKENS:
        return "fused_screen_kernel"
    if stage == "output" and tokens >= WIDE_OUTPUT_TOKENS:
        return "output_wide_kernel"
    return STAGE_KERNELS[stage]


SOURCE = os.path.join(ROOT, "calibration-free-moe_amd", "csrc", "cfmoe_reader.hip")
PROFILES = os.path.join(ROOT, "profiles")
PROBE_ELEMENTS = 1 << 27  # float32: 512 MiB read + 512 MiB written per probe launch


def source_digest() -> str:
    import hashlib

    with open(SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def stream_probe(device, steps: int = 10) -> dict:
    """A plain streaming kernel of known size (torch.neg over 512 MiB of float32).

    Its measured rate is the box's practical HBM bandwidth; under rocprofv3
    --pmc its FETCH_SIZE / WRITE_SIZE readings calibrate the counters.
    """
    src = torch.ones(PROBE_ELEMENTS, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    begin.record()
    for _ in range(steps):
        torch.neg(src, out=dst)
    end.record()
    torch.cuda.synchronize()
    seconds = begin.elapsed_time(end) * 1e-3 / steps
    moved = 2 * 4 * PROBE_ELEMENTS
    del src, dst
    torch.cuda.empty_cache()
    return {"kernel": "torch.neg float32", "bytes_per_launch": moved,
            "gbps": round(moved / seconds / 1e9, 1)}


def measured_traffic(kernel: str, config: str, tokens: int, layers: int) -> dict | None:
    """HBM bytes per launch of `kernel` from the committed counter summary.

    The summary (written by `bench.py --summarize`) holds FETCH_SIZE and
    WRITE_SIZE means per dispatch from two rocprofv3 --pmc runs, scaled by the
    same counters read on the streaming probe; it is used only when it was
    taken from the current kernel source on the same workload.
    """
    path = os.path.join(PROFILES, f"{kernel}.{config}_t{tokens}.pmc.txt")
    if not os.path.exists(path):
        return None
    fields = {}
    with open(path) as f:
        for line in f:
            key, sep, value = line.partition(":")
            if sep:
                fields[key.strip()] = value.strip()
    if fields.get("source_sha256_16") != source_digest():
        return None
    return {"bytes": float(fields["traffic_bytes_per_launch"]),
            "read_bytes": float(fields["read_bytes_per_launch"]),
            "write_bytes": float(fields["write_bytes_per_launch"]),
            "scale_read": float(fields["scale_read"]),
            "scale_write": float(fields["scale_write"]),
            "summary": os.path.relpath(path, ROOT)}


PILOT_SECONDS = 0.5  # the plan's pilot: replays per sample for about 0.5 s
PLAN_SAMPLES = 7     # samples whose median is reported


def time_graph(graph: torch.cuda.CUDAGraph, warmup: int, steps: int,
               sample_seconds: float = PILOT_SECONDS) -> dict:
    """Replay timings of a captured layer stack.

    After `warmup` untimed replays: (1) exactly `steps` replays, bracketed by
    synchronisations, give `ms_per_step` (their mean) and per-step event
    times; (2) the reference's measurement plan
    (scripts/speed_block.py:379-414): a pilot of about `sample_seconds`
    (PILOT_SECONDS by default) sizes a sample of `replays` replays, and the
    median of PLAN_SAMPLES such samples (each bracketed by events on the
    graph's stream) is `ms_median`. Profiler runs pass a shorter sample, so the
    trace holds fewer dispatch records.
    """
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = time.perf_counter()
    events = []
    for _ in range(steps):
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        graph.replay()
        end.record()
        events.append((begin, end))
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - start) * 1e3 / steps
    step_ms = [b.elapsed_time(e) for b, e in events]
    # pilot: whole replays until about sample_seconds have passed
    pilot, began = 0, time.perf_counter()
    while time.perf_counter() - began < sample_seconds:
        for _ in range(8):
            graph.replay()
        torch.cuda.synchronize()
        pilot += 8
    replays = max(1, round(pilot * sample_seconds / (time.perf_counter() - began)))
    samples = []
    for _ in range(PLAN_SAMPLES):
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(replays):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        samples.append(begin.elapsed_time(end) / replays)
    return {"ms_per_step": ms_per_step, "step_ms": step_ms, "ms_median": statistics.median(samples),
            "samples_ms": samples, "replays_per_sample": replays}


_WEIGHT_CACHE: dict[int, list] = {}


def layer_weights(name: str, layers: int, device) -> list:
    h, i, e, k, _, _, _, _, _ = CONFIGS[name]
    base = WEIGHT_SEEDS[name]
    cached = _WEIGHT_CACHE.get(base)
    if cached is None or len(cached) != layers:
        _WEIGHT_CACHE.clear()
        torch.cuda.empty_cache()
        started = time.perf_counter()
        cached = [device_weights(h, i, e, 32, seed=1000 * base + layer, device=device)
                  for layer in range(layers)]
        torch.cuda.synchronize()
        log(f"[{name}] generated {layers} layers in {time.perf_counter() - started:.1f}s")
        _WEIGHT_CACHE[base] = cached
    return cached


def shared_expert_us(name: str, stack: list, args, device) -> float | None:
    """Dense always-on shared expert beside the reader (C5), timed on its own.

    One BF16 SwiGLU MLP of width SHARED_WIDTH per layer on the same decode
    batch: gate/up [2W, H] and down [H, W] N(0, 0.02^2), computed dense with
    library GEMMs (hipBLASLt); its time is reported separately from the
    reader's, as the configuration asks.
    """
    width = SHARED_WIDTH.get(name)
    if width is None:
        return None
    h = CONFIGS[name][0]
    g = torch.Generator(device=device).manual_seed(5000)
    mlps = [((torch.randn(2 * width, h, generator=g, device=device) * 0.02).bfloat16(),
             (torch.randn(h, width, generator=g, device=device) * 0.02).bfloat16())
            for _ in stack]
    outs = [torch.empty_like(d["hidden"]) for _, d in stack]

    def run():
        for (gate_up, down), (_, d), out in zip(mlps, stack, outs):
            gu = d["hidden"] @ gate_up.T
            act = torch.nn.functional.silu(gu[:, :width]) * gu[:, width:]
            torch.matmul(act, down.T, out=out)

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    return time_graph(graph, args.warmup, args.steps, args.sample_seconds)["ms_median"] * 1e3 / len(stack)


def run_config(name: str, args, device) -> dict:
    h, i, e, k, layers, tokens, retention, keep, description = CONFIGS[name]
    layers = args.layers or layers
    tokens = args.tokens or tokens
    retention = getattr(args, "retention", 0.0) or retention
    keep = getattr(args, "keep", 0.0) or keep
    rank = 32
    plan = compile_budget(hidden_size=h, expert_width=i, top_k=k, retention=retention,
                          screen_keep=keep)
    log(f"[{name}] {layers} layers (H={h} I={i} E={e} K={k}) batch {tokens} "
        f"retention {retention} keep {keep}")
    weights = layer_weights(name, layers, device)
    workspace = ReaderWorkspace(plan, e, rank, tokens, device)
    stack = []
    for layer, w in enumerate(weights):
        reader = ProgressiveReader(
            w["gate_up"], w["down"], w["encoder"], w["decoder"], plan, tokens,
            sketch=w["sketch"], selection_score="point", workspace=workspace,
        )
        stack.append((reader, device_inputs(w, tokens, k, seed=7919 * layer + tokens, device=device,
                                            zipf=ZIPF.get(name))))
    torch.cuda.synchronize()
    for reader, d in stack:
        reader(d["hidden"], d["ids"], d["weights"], out=d["out"])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for reader, d in stack:
            reader(d["hidden"], d["ids"], d["weights"], out=d["out"])
    timing = time_graph(graph, args.warmup, args.steps, args.sample_seconds)
    ms_per_step = timing["ms_per_step"]
    us_per_layer = timing["ms_median"] * 1e3 / layers
    log(f"[{name}] {us_per_layer:.2f} us/layer (median of {PLAN_SAMPLES} samples of "
        f"{timing['replays_per_sample']} replays; {ms_per_step:.3f} ms/step over {args.steps} steps)")
    # algorithmic bytes of each layer call, from that layer's own routes and selections
    byte_rows = []
    for reader, d in stack:
        reader(d["hidden"], d["ids"], d["weights"], out=d["out"])
        torch.cuda.synchronize()
        byte_rows.append(algorithmic_bytes(reader, tokens))
    mean_bytes = {key: float(np.mean([row[key] for row in byte_rows])) for key in byte_rows[0]}
    # live per-stage timing: each stage relaunched over the whole stack in a graph
    stage_us = {}
    repeats = 4
    for stage in _ext.STAGES:
        # the shared workspace holds one complete call's state (the last
        # layer's) when a stage is relaunched over the stack
        last_reader, last = stack[-1]
        last_reader(last["hidden"], last["ids"], last["weights"], out=last["out"])
        torch.cuda.synchronize()
        stage_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(stage_graph):
            for _ in range(repeats):
                for reader, d in stack:
                    reader.launch_stage(stage, d["hidden"], d["ids"], d["weights"], None, d["out"])
        stage_graph.replay()
        torch.cuda.synchronize()
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        stage_graph.replay()
        end.record()
        torch.cuda.synchronize()
        stage_us[stage] = begin.elapsed_time(end) * 1e3 / (repeats * layers)
    shared_us = shared_expert_us(name, stack, args, device)
    dominant = max(STAGE_BYTES, key=lambda s: stage_us[s])
    dominant_bytes = sum(mean_bytes[key] for key in stage_bytes(dominant, tokens, rank))
    achieved = dominant_bytes / (stage_us[dominant] * 1e-6) / 1e9
    return {
        "name": name,
        "description": description,
        "layers": layers,
        "tokens": tokens,
        "retention": retention,
        "screen_keep": keep,
        "zipf": ZIPF.get(name),
        "shared_expert_us_per_layer": shared_us,
        "final_count": plan.final_count,
        "ms_per_step": ms_per_step,
        "us_per_layer": us_per_layer,
        "us_per_layer_steps": ms_per_step * 1e3 / layers,
        "us_per_layer_median_event": statistics.median(timing["step_ms"]) * 1e3 / layers,
        "replays_per_sample": timing["replays_per_sample"],
        "tokens_per_s": tokens * 1e6 / (us_per_layer * layers),
        "layer_tokens_per_s": tokens * 1e6 / us_per_layer,
        "bytes_per_layer": mean_bytes,
        "achieved_gbps": mean_bytes["total"] / (us_per_layer * 1e-6) / 1e9,
        "layer_roofline_frac": mean_bytes["total"] / (us_per_layer * 1e-6) / 1e9 / HBM_PEAK_GBPS,
        "stage_us": stage_us,
        "dominant": dominant,
        "dominant_bytes": dominant_bytes,
        "dominant_gbps": achieved,
    }


def cpu_threads() -> int:
    """Threads of this process's CPU share: the affinity set, at most the
    OpenMP thread setting of the box (16 per GPU)."""
    available = len(os.sched_getaffinity(0))
    return max(1, min(available, int(os.environ.get("OMP_NUM_THREADS") or available)))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float) -> dict:
    """The CPU oracle (C, OpenMP over the CPU share) on the C1 layer: OLMoE
    shape, batch 1; two warm-up calls, then the median of at least ten over
    about `seconds`."""
    from oracle import oracle
    from tests.synthetic import bits

    h, i, e, k = 2048, 1024, 64, 8
    plan = compile_budget(hidden_size=h, expert_width=i, top_k=k, retention=0.123,
                          screen_keep=0.625)
    data = device_layer(h, i, e, k, 32, 1, seed=1000 * 1, device=torch.device("cuda:0"))
    codes, stats = data["sketch"]
    down = data["down"]
    weights = oracle.Weights(
        gate_up=bits(data["gate_up"]),
        down=bits(down.transpose(1, 2)),
        codes=codes.cpu().contiguous().numpy(),
        stats=bits(stats.permute(0, 2, 3, 1).contiguous()),
        norms=down.float().square().sum(1).sqrt().cpu().contiguous().numpy(),
        signs=block_hadamard_signs(h, "cpu").numpy(),
        encoder_t=bits(data["encoder"].transpose(1, 2).contiguous()),
        decoder=bits(data["decoder"]),
    )
    x = bits(data["hidden"])
    ids = data["ids"].cpu().numpy()
    w = data["weights"].cpu().numpy()
    threads = cpu_threads()
    runs = []
    for _ in range(2):
        oracle.forward(weights, x, ids, w, final_count=plan.final_count, keep=80, threads=threads)
    deadline = time.perf_counter() + seconds
    while time.perf_counter() < deadline or len(runs) < 10:
        begin = time.perf_counter()
        oracle.forward(weights, x, ids, w, final_count=plan.final_count, keep=80, threads=threads)
        runs.append(time.perf_counter() - begin)
    return {
        "value": statistics.median(runs) * 1e6,
        "unit": "us/layer",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "logical_cpus_visible": os.cpu_count(),
        "sample": f"C1 OLMoE-shaped layer, batch 1, median of {len(runs)} oracle calls "
                  f"after 2 warm-ups ({threads} OpenMP threads)",
        "gbps_on_algorithmic_bytes": 17_804_352 / statistics.median(runs) / 1e9,
    }


def _short_name(name: str) -> str:
    return name.split("(")[0].split("<")[0].split("::")[-1].strip() or name[:60]


def _rocprof_rows(directory: str, suffix: str) -> list[dict]:
    import csv
    import glob

    rows = []
    for path in sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True)):
        with open(path) as f:
            rows += list(csv.DictReader(f))
    return rows


def summarize_trace(directory: str, command: str) -> str:
    """Per-kernel launch statistics of a rocprofv3 --kernel-trace --stats run."""
    durations: dict[str, list[int]] = {}
    reader_kernels = set(STAGE_KERNELS.values()) | {"select_all_kernel", "group_exact_kernel",
                                                     "fused_screen_kernel", "output_wide_kernel",
                                                     "output_staged_kernel", "select_exact_kernel"}
    for row in _rocprof_rows(directory, "kernel_trace.csv"):
        name = _short_name(row["Kernel_Name"])
        if name not in reader_kernels:
            continue  # setup work (weight generation, recovery bank, probe)
        durations.setdefault(name, []).append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    lines = [f"command: {command}", f"source_sha256_16: {source_digest()}", "",
             f"{'kernel':34s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'total_ms':>10s}"]
    for name, values in sorted(durations.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{name:34s} {len(values):7d} {sum(values) / len(values) / 1e3:9.2f} "
                     f"{min(values) / 1e3:9.2f} {max(values) / 1e3:9.2f} {sum(values) / 1e6:10.3f}")
    return "\n".join(lines) + "\n"


def summarize_pmc(fetch_dir: str, write_dir: str, kernel: str, command: str) -> str:
    """HBM traffic per launch of `kernel` from FETCH_SIZE and WRITE_SIZE passes.

    Both counters are in KiB per dispatch; each is scaled by the ratio of the
    streaming probe's known bytes to what the same counter read for it.
    """
    def means(directory: str, counter: str) -> dict[str, float]:
        values: dict[str, list[float]] = {}
        for row in _rocprof_rows(directory, "counter_collection.csv"):
            if row["Counter_Name"] != counter:
                continue
            values.setdefault(_short_name(row["Kernel_Name"]), []).append(float(row["Counter_Value"]))
        return {name: sum(v) / len(v) for name, v in values.items()}

    fetch, write = means(fetch_dir, "FETCH_SIZE"), means(write_dir, "WRITE_SIZE")
    probe = next(name for name in fetch if "neg" in name or "elementwise" in name)
    known = 4.0 * PROBE_ELEMENTS
    scale_read = known / (fetch[probe] * 1024.0)
    scale_write = known / (write[probe] * 1024.0)
    read = fetch[kernel] * 1024.0 * scale_read
    written = write[kernel] * 1024.0 * scale_write
    lines = [
        f"command: {command}",
        f"source_sha256_16: {source_digest()}",
        f"kernel: {kernel}",
        f"fetch_kib_per_launch: {fetch[kernel]:.1f}",
        f"write_kib_per_launch: {write[kernel]:.1f}",
        f"probe_kernel: {probe}",
        f"probe_fetch_kib: {fetch[probe]:.1f}",
        f"probe_write_kib: {write[probe]:.1f}",
        f"probe_known_bytes_each_way: {known:.0f}",
        f"scale_read: {scale_read:.4f}",
        f"scale_write: {scale_write:.4f}",
        f"read_bytes_per_launch: {read:.0f}",
        f"write_bytes_per_launch: {written:.0f}",
        f"traffic_bytes_per_launch: {read + written:.0f}",
        "",
        "all kernels (KiB per dispatch, unscaled):",
    ]
    for name in sorted(fetch):
        lines.append(f"  {name:34s} FETCH_SIZE {fetch[name]:14.1f}  WRITE_SIZE {write.get(name, 0.0):14.1f}")
    return "\n".join(lines) + "\n"


def main() -> int:
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize":
        # bench.py --summarize trace DIR OUT COMMAND
        # bench.py --summarize pmc FETCH_DIR WRITE_DIR KERNEL OUT COMMAND
        mode = sys.argv[2]
        if mode == "trace":
            text = summarize_trace(sys.argv[3], sys.argv[5])
            out = sys.argv[4]
        else:
            text = summarize_pmc(sys.argv[3], sys.argv[4], sys.argv[5], sys.argv[7])
            out = sys.argv[6]
        with open(out, "w") as f:
            f.write(text)
        print(text)
        return 0
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=4)
    parser.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    parser.add_argument("--layers", type=int, default=0)
    parser.add_argument("--tokens", type=int, default=0)
    parser.add_argument("--extra",
                        default="c1:1,c3:1,c3:32,c3:128,c4:256,c4:256:0.06,c4:256:0.25,"
                                "c5:1,c5:128,c5:1:0.123:1.0,c5:128:0.123:1.0",
                        help="comma list of config:tokens[:retention[:screen_keep]] "
                             "measured beside the headline")
    parser.add_argument("--retention", type=float, default=0.0,
                        help="the headline configuration's retention (0: the configuration's own)")
    parser.add_argument("--keep", type=float, default=0.0,
                        help="the headline configuration's screen keep (0: the configuration's own)")
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--sample-seconds", type=float, default=PILOT_SECONDS,
                        help="length of each timing sample (shorter under a profiler)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this reader runs without collectives; got --gpus {args.gpus}",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    _ext.library()
    headline = run_config(args.config, args, device)
    extras = []
    for item in filter(None, args.extra.split(",")):
        name, *fields = item.split(":")
        sub = argparse.Namespace(**vars(args))
        sub.layers = 0
        sub.tokens = int(fields[0]) if fields and fields[0] else 0
        sub.retention = float(fields[1]) if len(fields) > 1 else 0.0
        sub.keep = float(fields[2]) if len(fields) > 2 else 0.0
        torch.cuda.empty_cache()
        extras.append(run_config(name, sub, device))
    probe = stream_probe(device)
    baseline = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None
    h, i, e, k, layers, tokens, _, _, description = CONFIGS[args.config]
    retention, keep = headline["retention"], headline["screen_keep"]
    kernel = stage_kernel(headline["dominant"], headline["tokens"])
    traffic = measured_traffic(kernel, args.config, headline["tokens"], headline["layers"])
    line = {
        "metric": METRIC,
        "value": round(headline["us_per_layer"], 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(headline["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init BF16 weights, seeded router and hidden states)",
        "config": {
            "workload": f"{args.config}: {description}",
            "hidden": h, "expert_width": i, "experts": e, "top_k": k,
            "layers": headline["layers"], "batch": headline["tokens"],
            "retention": retention, "screen_keep": keep, "rank": 32,
            "selection_score": "point", "final_count": headline["final_count"],
        },
        "timing": {
            "value": f"median of {PLAN_SAMPLES} samples after the {args.warmup} warm-up replays, each "
                     f"sample {headline['replays_per_sample']} graph replays sized by a pilot of "
                     f"about {args.sample_seconds} s (the reference's measurement plan, "
                     "scripts/speed_block.py:379-414), divided by the layers",
            "ms_per_step": f"mean of exactly {args.steps} replays between synchronisations",
            "stage_us": "each stage relaunched alone (cfmoe_launch_stage) 4 times over the stack's "
                        "layers in one HIP graph, after one full call of the last layer: every "
                        "relaunch reads the workspace that call left (the score stage, and the "
                        "encode stage at rank 32, launch nothing; up to four tokens the layer "
                        "runs select and exact as one launch, relaunched here as their separate "
                        "kernels); timing only",
        },
        "us_per_layer_steps": round(headline["us_per_layer_steps"], 3),
        "us_per_layer_median_step": round(headline["us_per_layer_median_event"], 3),
        "tokens_per_s": round(headline["tokens_per_s"], 1),
        "achieved_gbps": round(headline["achieved_gbps"], 1),
        "algorithmic_bytes_per_layer": headline["bytes_per_layer"],
        "stage_us": {s: round(v, 3) for s, v in headline["stage_us"].items()},
        "roofline": {
            "bound": "hbm",
            "kernel": kernel,
            "algorithmic_bytes_per_launch": round(headline["dominant_bytes"]),
            "launch_us": round(headline["stage_us"][headline["dominant"]], 3),
            "achieved": round(headline["dominant_gbps"], 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(headline["dominant_gbps"] / HBM_PEAK_GBPS, 4),
            "traffic": None if traffic is None else round(traffic["bytes"]),
            "traffic_detail": traffic,
            "layer_frac": round(headline["layer_roofline_frac"], 4),
        },
        "stream_probe": probe,
        "cpu_baseline": baseline,
        "extra": [
            {key: (round(v, 3) if isinstance(v, float) else v) for key, v in x.items()
             if key in ("name", "description", "layers", "tokens", "retention", "screen_keep",
                        "zipf", "final_count", "us_per_layer", "tokens_per_s", "achieved_gbps",
                        "layer_roofline_frac", "dominant", "dominant_gbps", "stage_us",
                        "shared_expert_us_per_layer", "us_per_layer_median_event",
                        "us_per_layer_steps")}
            for x in extras
        ],
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
