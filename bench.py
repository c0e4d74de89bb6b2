"""Benchmark of the hip backend on one MI355X: every BASELINE configuration in one JSON line.

Headline (``value``): the fused-kernel HBM throughput of BASELINE config C2 - the fp32 bandwidth graph
``softmax(tanh(x*0.5+y)*sigmoid(y) - exp(clamp(x,-8,8))*1e-3, -1)`` over x, y in U(-4, 4) [16384, 8192]
(generator seed 1, x then y) compiled with ``chroma_amd.compile(..., backend="hip")``. One step is one
execution of the compiled program on inputs already resident in HBM; GB/s counts the algorithmic bytes
(read x, read y, write the output: 3 x 16384 x 8192 x 4 = 1,610,612,736 B per step).

Beside it the same line reports:

* ``roofline``: the C2 kernel's algorithmic bytes over its average duration from hipEvents recorded on
  the runtime's own stream around the timed launches, against MI355X's 8 TB/s; ``traffic`` comes from
  the committed rocprofv3 FETCH_SIZE/WRITE_SIZE measurement (profiles/) when present;
* ``cpu_baseline``: the CPU restatement of Chroma's CPU backend (oracle/, one thread) timed on this host
  on a bounded sample of the same graph;
* ``hbm_copy``: a plain copy kernel's GB/s, the practical HBM ceiling the fractions can be read against;
* ``rows``: row reductions (RMSNorm, softmax, log-sum-exp) at the widths of C1, C5 and the vocabulary;
* ``c1``: the MLP block; ``dev_forward`` (C3) and ``decode`` (C4): the dev MoE model's 8-token forward and
  256-position KV-cached decode, end to end (host arrays in and out) in the reference's interleaved
  method, with device-only times and rooflines; ``c5``: the GPT-OSS-20B-shaped bf16 model's 2048-token
  prefill (matrix-core fraction on the work actually performed) and its decode step at a full
  4096-position cache (HBM fraction), with the oracle's time and parity on a reduced slice;
* ``host``: CPU model, core counts, ROCm version and GPU name.

``--only experts`` (not in the default line) times the C5 expert products alone against the vendor
library's dense, grouped and per-expert GEMMs of the same FLOPs.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import random
import statistics
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "dev-model 8-tok fwd ms; 256-KV decode ms; fused-kernel HBM GB/s"
C2_SHAPE = (16384, 8192)
C2_BYTES = 3 * C2_SHAPE[0] * C2_SHAPE[1] * 4
C1_BYTES = 3 * 4096 * 1024 * 4 + 2 * 8 * 1024 * 4
C1_FLOPS = 2 * 8 * 1024 * 4096 * 3
# C3: unembedding 102,957,056 + 12 x (dense 155,856 + all 12 experts' weights and biases 2,377,728)
# + embedding rows 4,096 + logits 6,434,816.
C3_BYTES = 102_957_056 + 12 * (155_856 + 2_377_728) + 4_096 + 6_434_816
# C4 step: unembedding + 12 x (dense + 4 selected experts x (131,072 + 1,024 + 65,536 + 512)) + K/V cache
# 393,216 + one logits row 804,352.
C4_BYTES = 102_957_056 + 12 * (155_856 + 4 * (131_072 + 1_024 + 65_536 + 512)) + 393_216 + 804_352
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = ROOT / "profiles" / "c2_fused_softmax_traffic.txt"
C5_DECODE_TRAFFIC_FILE = ROOT / "profiles" / "c5_decode_traffic.txt"
ROWS_TRAFFIC_FILE = ROOT / "profiles" / "row_reductions_traffic.txt"
SMALL_TRAFFIC_FILE = ROOT / "profiles" / "c1_c3_c4_traffic.txt"
C5_PREFILL_COUNTERS_FILE = ROOT / "profiles" / "c5_prefill_mfma_counters.txt"
VOCAB = 201088


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def host_info() -> dict:
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    rocm = "unknown"
    for candidate in (Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / ".info" / "version",):
        if candidate.exists():
            rocm = candidate.read_text().strip()
    import torch

    return {
        "cpu_model": model,
        "nproc": os.cpu_count(),
        "cpus_available": len(os.sched_getaffinity(0)),
        "rocm": rocm,
        "torch": torch.__version__,
        "python": platform.python_version(),
        "oracle_threads": 1,
    }


def roofline(amount: float, ms: float, bound: str = "hbm", traffic=None) -> dict:
    """Achieved rate of ``amount`` bytes (hbm) or flops (mfma) in ``ms`` against MI355X's peak."""
    if bound == "hbm":
        achieved = amount / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}
    achieved = amount / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": traffic}


def device_ms(program, runs: int, warmup: int = 3) -> float:
    """Average time of one execution of ``program``'s plan on what its staging regions hold, from hipEvents
    on the runtime's stream around ``runs`` back-to-back executions."""
    native = program.native
    native.execute(warmup)
    return native.execute(runs, timed=True) / runs


def chained_ms(program, copies: int, iterations: int) -> float:
    """Time of one execution of ``program``'s plan from hipEvents around ``iterations`` launches of one graph
    holding ``copies`` back-to-back executions: each kernel's own time plus the dispatch barrier in front of
    it, without the host's per-replay graph launch (~10 us), which would otherwise set a one-kernel plan."""
    native = program.native
    native.execute(1)
    return native.execute_chained(copies, iterations)


def plan_kernels(directory: Path) -> list:
    """Kernel names of a compiled artifact's launches, in order (from its model.plan)."""
    return [line.split()[1] for line in (directory / "model.plan").read_text().splitlines() if line.startswith("launch ")]


def interleaved(calls: dict, warmup: int = 10, runs: int = 100, rounds: int = 2, seed: int = 0) -> dict:
    """The reference's timing method (scripts/benchmark.py:221-230, docs/benchmarks.md:12-16): every call
    once per round in a seeded shuffled order, ``warmup`` untimed rounds, then ``runs`` timed rounds;
    repeated ``rounds`` times and pooled; median, p10 and p90 in ms."""
    samples = {name: [] for name in calls}
    rng = random.Random(seed)
    order = list(calls)
    for _ in range(rounds):
        for _ in range(warmup):
            rng.shuffle(order)
            for name in order:
                calls[name]()
        for _ in range(runs):
            rng.shuffle(order)
            for name in order:
                start = time.perf_counter()
                calls[name]()
                samples[name].append((time.perf_counter() - start) * 1e3)
    out = {}
    for name, values in samples.items():
        values.sort()
        out[name] = {"median_ms": round(statistics.median(values), 4), "p10_ms": round(values[len(values) // 10], 4),
                     "p90_ms": round(values[len(values) * 9 // 10], 4), "samples": len(values)}
    return out


def timed(call, warmup: int, runs: int) -> dict:
    for _ in range(warmup):
        call()
    samples = []
    for _ in range(runs):
        start = time.perf_counter()
        call()
        samples.append((time.perf_counter() - start) * 1e3)
    samples.sort()
    return {"median_ms": round(statistics.median(samples), 4), "p10_ms": round(samples[len(samples) // 10], 4), "runs": runs}


def read_traffic(path: Path = TRAFFIC_FILE, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch (per step for C5 decode, per execution of a plan elsewhere) from a committed
    rocprofv3 counter summary (the line ``<key> <bytes>``), or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(key + " ") and line[len(key) + 1 :].strip().replace(".", "", 1).isdigit():
            return int(float(line.split()[-1]))
    return None


# ----------------------------------------------------------------------------------------- C2 (headline)
def bench_c2(args, work: Path) -> dict:
    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd.models.blocks import BandwidthGraph, bandwidth_inputs

    x, y = bandwidth_inputs()
    exported = torch.export.export(BandwidthGraph(), (x, y))
    log("compiling C2 for hip")
    program = chroma_amd.compile(exported, work / "c2")
    native = program.native
    native.upload([x.numpy(), y.numpy()])
    native.execute(max(args.warmup, 1))
    # Timed region: K steps on device-resident inputs; execute() synchronizes the runtime stream.
    start = time.perf_counter()
    event_ms = native.execute(args.steps, timed=True)
    wall = time.perf_counter() - start
    output = np.empty(C2_SHAPE, dtype=np.float32)
    native.download([output])
    sums = output[::1024].sum(axis=1)
    if not np.allclose(sums, 1.0, rtol=1e-4):
        raise RuntimeError(f"C2 rows do not sum to 1: {sums[:4]}")
    kernel_ms = event_ms / args.steps
    end_to_end = timed(lambda: program(x.numpy(), y.numpy()), 1, 3)
    device = native.device
    program.close()
    return {
        "value": C2_BYTES * args.steps / wall / 1e9,
        "ms_per_step": wall / args.steps * 1e3,
        "kernel_ms": kernel_ms,
        "roofline": roofline(C2_BYTES, kernel_ms, traffic=read_traffic()),
        "stats": program.stats,
        "end_to_end_ms": end_to_end,
        "device": device,
    }


def cpu_c2(work: Path) -> dict:
    """The oracle on a bounded sample of C2 (the first rows), one thread."""
    import torch

    from chroma_amd.models.blocks import BandwidthGraph, bandwidth_inputs
    from oracle import compile_cpu

    rows = 2048
    x, y = bandwidth_inputs()
    x, y = x[:rows].contiguous(), y[:rows].contiguous()
    program = compile_cpu(torch.export.export(BandwidthGraph(), (x, y)), work / "c2_cpu")
    arrays = (x.numpy(), y.numpy())
    program(*arrays)
    times = []
    deadline = time.perf_counter() + 12.0
    while time.perf_counter() < deadline or len(times) < 2:
        start = time.perf_counter()
        program(*arrays)
        times.append(time.perf_counter() - start)
    seconds = statistics.median(times)
    sample_bytes = 3 * rows * C2_SHAPE[1] * 4
    program.close()
    return {
        "value": round(sample_bytes / seconds / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"C2 graph on the first {rows} of 16384 rows ([{rows},8192] x2 fp32), median of {len(times)} runs, "
        f"{seconds * 1e3:.1f} ms each; oracle = CPU restatement of Chroma's CPU backend, -O3 -ffp-contract=off, 1 thread",
    }


# ------------------------------------------------------------------------------- HBM ceiling and rows
def bench_copy(work: Path) -> dict:
    """A plain copy over [16384, 8192] fp32 (512 MiB read + 512 MiB written per launch)."""
    import torch

    import chroma_amd
    from chroma_amd.models.blocks import Copy, bandwidth_inputs

    x = bandwidth_inputs()[0]
    with chroma_amd.compile(torch.export.export(Copy(), (x,)), work / "copy") as program:
        program.native.upload([x.numpy()])
        ms = device_ms(program, 20)
    moved = 2 * x.numel() * 4
    return {"workload": "x * 1.0 over [16384, 8192] fp32", "bytes": moved, "ms": round(ms, 4), "gbs": round(moved / (ms * 1e-3) / 1e9, 1),
            "frac_of_peak": round(moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


ROW_CASES = [
    ("rmsnorm", 2048, 1024), ("rmsnorm", 2048, 2880), ("rmsnorm", 8, VOCAB), ("rmsnorm", 2048, VOCAB),
    ("softmax", 8, VOCAB), ("softmax", 2048, VOCAB), ("logsumexp", 8, VOCAB), ("logsumexp", 2048, VOCAB),
]


def row_case_module(kind: str, rows: int, width: int):
    import torch

    from chroma_amd.models.blocks import RowLogSumExp, RowNorm, RowSoftmax

    x = torch.randn(rows, width, generator=torch.Generator().manual_seed(0))
    module = RowNorm(width) if kind == "rmsnorm" else RowSoftmax() if kind == "softmax" else RowLogSumExp()
    return module, x


def bench_rows(work: Path, cpu: bool) -> list:
    """Row reductions in fp32, x ~ N(0, 1) seed 0, inputs resident: time per execution (``chained_ms``) and
    GB/s on the algorithmic bytes (read + write of R x D for RMSNorm and softmax, read + R floats for
    log-sum-exp), ``traffic`` from the committed counter summary, checked against the oracle on the first
    rows; the oracle's time on a sample of at most 64 rows."""
    import shutil

    import numpy as np
    import torch

    import chroma_amd
    from oracle import compile_cpu

    results = []
    for kind, rows, width in ROW_CASES:
        module, x = row_case_module(kind, rows, width)
        moved = rows * width * 4 + (rows * 4 if kind == "logsumexp" else rows * width * 4)
        with chroma_amd.compile(torch.export.export(module, (x,)), work / f"{kind}_{rows}_{width}") as program:
            program.native.upload([x.numpy()])
            small = rows * width < (1 << 26)
            ms = chained_ms(program, 20 if small else 5, 10 if small else 3)
            replay = device_ms(program, 20 if small else 5)
            got = program(x.numpy())
            launches = program.stats["launches"]
        sample = min(rows, 64)
        head = x[:sample].contiguous()
        case = f"{kind} [{rows},{width}]"
        entry = {"kind": kind, "shape": [rows, width], "dtype": "f32", "launches": launches, "ms": round(ms, 4),
                 "replay_ms": round(replay, 4), "algorithmic_bytes": moved,
                 "roofline": roofline(moved, ms, traffic=read_traffic(ROWS_TRAFFIC_FILE, f"traffic_bytes_per_execution {case}"))}
        if cpu:
            oracle = compile_cpu(torch.export.export(module, (head,)), work / f"{kind}_{rows}_{width}_cpu")
            want = oracle(head.numpy())
            np.testing.assert_allclose(got[:sample], want, rtol=1e-4, atol=1e-5)
            cpu_ms = timed(lambda: oracle(head.numpy()), 1, 3)["median_ms"]
            oracle.close()
            sample_bytes = sample * width * 4 + (sample * 4 if kind == "logsumexp" else sample * width * 4)
            entry["cpu_oracle"] = {"rows": sample, "ms": cpu_ms, "gbs": round(sample_bytes / (cpu_ms * 1e-3) / 1e9, 3)}
        results.append(entry)
        log(f"{kind} [{rows},{width}] {ms * 1e3:.1f} us, {entry['roofline']['achieved']} GB/s")
        shutil.rmtree(work / f"{kind}_{rows}_{width}", ignore_errors=True)
    return results


# ------------------------------------------------------------------------------------------------- C1
def bench_c1(work: Path, cpu: bool) -> dict:
    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd.models.blocks import mlp_block, mlp_inputs
    from oracle import compile_cpu

    module, (x,) = mlp_block(), mlp_inputs()
    exported = torch.export.export(module, (x,))
    program = chroma_amd.compile(exported, work / "c1")
    array = x.numpy()
    got = program(array)
    program.native.upload([array])
    ms = chained_ms(program, 20, 10)
    result = {"workload": "MLP block x[8,1024] fp32 seed 0: RMSNorm, SiLU(gate)*up (1024->4096), down (4096->1024), residual; weights N(0,0.02) seed 0",
              "device_ms": round(ms, 4), "replay_ms": round(device_ms(program, 50), 4), "launches": program.stats["launches"],
              "algorithmic_bytes": C1_BYTES, "flops": C1_FLOPS,
              "roofline": roofline(C1_BYTES, ms, traffic=read_traffic(SMALL_TRAFFIC_FILE, "traffic_bytes_per_execution c1")),
              "host_to_host": timed(lambda: program(array), 10, 100)}
    if cpu:
        oracle = compile_cpu(exported, work / "c1_cpu")
        np.testing.assert_allclose(got, oracle(array), rtol=1e-4, atol=1e-5)
        result["cpu_oracle"] = timed(lambda: oracle(array), 2, 20)
        oracle.close()
    program.close()
    return result


# ------------------------------------------------------------------------------------------------- C3
def bench_dev(work: Path, cpu: bool) -> dict:
    """C3: the dev model's 8-token fp32 forward, host arrays in and out, interleaved with the oracle."""
    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd.models.dev import make_dev_model, weights_digest
    from oracle import compile_cpu

    model = make_dev_model(0)
    tokens = torch.randint(0, VOCAB, (8,), generator=torch.Generator().manual_seed(0))
    exported = torch.export.export(model, (tokens,))
    log("compiling the dev model for hip and the oracle")
    program = chroma_amd.compile(exported, work / "dev")
    oracle = compile_cpu(exported, work / "dev_cpu") if cpu else None
    array = tokens.numpy()
    got = program(array)
    result = {"workload": "dev MoE model (12 layers, 59,079,408 params, vocab 201088), 8-token fp32 forward, batch 1, tokens ~U[0,201088) seed 0",
              "weights_sha256": weights_digest(model), "launches": program.stats["launches"]}
    if oracle is not None:
        want = oracle(array)
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
        result["argmax_equal"] = bool((got.argmax(-1) == want.argmax(-1)).all())
    out = program(array)  # the reference's out= method reuses an earlier result (scripts/benchmark.py:207-208)
    calls = {"hip_fresh": lambda: program(array), "hip_reuse": lambda: program(array, out=out)}
    if oracle is not None:
        calls["cpu_oracle"] = lambda: oracle(array)
    timings = interleaved(calls, warmup=10, runs=100, rounds=2)
    result.update(timings)
    result["method"] = "2 rounds x (10 warmup + 100 timed) of seeded interleaved calls, pooled (scripts/benchmark.py:221-230)"
    program.native.upload([array])
    ms = device_ms(program, 100, warmup=5)
    result["hip_device_ms"] = round(ms, 4)
    result["roofline"] = roofline(C3_BYTES, ms, traffic=read_traffic(SMALL_TRAFFIC_FILE, "traffic_bytes_per_execution dev"))
    result["algorithmic_bytes"] = C3_BYTES
    program.close()
    if oracle is not None:
        oracle.close()
    return result


# ------------------------------------------------------------------------------------------------- C4
def bench_decode(work: Path, steps: int, cpu: bool) -> dict:
    """C4: the dev model's KV-cached decode at a 256-position cache through ``Decoder`` (host mask and cache
    work included), the padded uncached 256-token graph and a 32-token prefill through the 256-step graph,
    each beside the oracle; plus the decode step's device-only time and roofline."""
    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd import Decoder
    from chroma_amd.models.cached import export_cached, export_uncached
    from chroma_amd.models.dev import make_dev_model
    from oracle import compile_cpu

    model = make_dev_model(0)
    graphs = {"prefill": export_cached(model, 256, 256), "decode": export_cached(model, 256, 1), "full": export_uncached(model, 256)}
    log("compiling the decode graphs for hip and the oracle")
    hip = {name: chroma_amd.compile(graph, work / f"hip_{name}") for name, graph in graphs.items()}
    cpu_programs = {name: compile_cpu(graph, work / f"cpu_{name}") for name, graph in graphs.items()} if cpu else {}
    tokens = torch.randint(0, VOCAB, (32 + steps,), generator=torch.Generator().manual_seed(0)).numpy()
    results = {"workload": "dev model, Decoder(export_cached(m,256,256), export_cached(m,256,1)); prefill 8 tokens ~U[0,201088) seed 0, "
               f"then {steps} single-token steps; 32-token prefill through the 256-step graph; padded export_uncached(m,256)"}
    padded = np.zeros(256, dtype=np.int64)
    padded[:16] = tokens[:16]
    last = np.array([15], dtype=np.int64)
    for name, programs in (("hip", hip), ("cpu_oracle", cpu_programs)):
        if not programs:
            continue
        decoder = Decoder(programs["prefill"], programs["decode"])
        count = steps if name == "hip" else min(steps, 32)
        rounds, samples = (3 if name == "hip" else 1), []
        for _ in range(rounds):
            decoder.reset()
            decoder.append(tokens[:8])
            for i in range(8, 8 + count):
                start = time.perf_counter()
                decoder.append(tokens[i : i + 1])
                samples.append((time.perf_counter() - start) * 1e3)
        prefill = []
        for _ in range(10 if name == "hip" else 3):
            decoder.reset()
            start = time.perf_counter()
            decoder.append(tokens[:32])
            prefill.append((time.perf_counter() - start) * 1e3)
        entry = {"decode_step": {"median_ms": round(statistics.median(samples), 4), "steps": len(samples)},
                 "prefill_32": {"median_ms": round(statistics.median(prefill), 4), "runs": len(prefill)},
                 "uncached_256": timed(lambda: programs["full"](padded, last), 2, 10 if name == "hip" else 3)}
        if name == "hip":
            decoder.reset()
            decoder.append(tokens[:8])
            decoder.greedy(tokens[8:9])  # compiles the selection program
            greedy = []
            for i in range(9, 8 + count):
                start = time.perf_counter()
                decoder.greedy(tokens[i : i + 1])
                greedy.append((time.perf_counter() - start) * 1e3)
            entry["decode_step_greedy"] = {"median_ms": round(statistics.median(greedy), 4), "steps": len(greedy)}
            # device-only decode step: the decode plan on what its staging holds after the last step
            ms = device_ms(programs["decode"], 100, warmup=5)
            entry["decode_step_device_ms"] = round(ms, 4)
            entry["roofline"] = roofline(C4_BYTES, ms, traffic=read_traffic(SMALL_TRAFFIC_FILE, "traffic_bytes_per_execution decode"))
            entry["algorithmic_bytes_per_step"] = C4_BYTES
        decoder.close()
        results[name] = entry
    if cpu:
        np.testing.assert_allclose(hip["full"](padded, last), cpu_programs["full"](padded, last), rtol=1e-4, atol=1e-5)
    for program in (*hip.values(), *cpu_programs.values()):
        program.close()
    return results


# ------------------------------------------------------------------------------------------------- C5
C5_CONTEXT, C5_PREFILL = 4096, 2048


def c5_live_flops(config, tokens: int) -> dict:
    """Multiply-add work (2 flops each) of one fresh ``export_cached(m, context, tokens)`` prefill as it
    must be performed: the projections, the four selected experts per token, the attention over the query
    -key pairs the masks leave live (causal on full layers, the last ``sliding_window`` keys on window
    layers; cached keys are all masked at a fresh prefill) and one unembedded row."""
    d, hd, heads, kv = config.hidden_size, config.head_dim, config.num_attention_heads, config.num_key_value_heads
    inter, top, layers = config.intermediate_size, config.experts_per_token, config.num_hidden_layers
    window = config.sliding_window
    full_pairs = tokens * (tokens + 1) // 2
    window_pairs = sum(min(t + 1, window) for t in range(tokens))
    flops = {
        "qkv": 2 * tokens * d * hd * (heads + 2 * kv) * layers,
        "out": 2 * tokens * hd * heads * d * layers,
        "router": 2 * tokens * d * config.num_experts * layers,
        "experts_up": 2 * tokens * top * 2 * inter * d * layers,
        "experts_down": 2 * tokens * top * d * inter * layers,
        # QK^T and PV: 4 * head_dim flops per live pair and query head; even layers use the window
        "attention": 4 * hd * heads * (full_pairs * (layers // 2) + window_pairs * (layers - layers // 2)),
        "unembedding": 2 * d * config.vocab_size,
    }
    flops["total"] = sum(flops.values())
    return flops


def c5_decode_bytes(config, cached: int) -> int:
    """HBM bytes one decode step must read with ``cached`` valid cache positions: every dense weight, the
    four selected experts of every layer (bf16 weights and biases), the unembedding, and the live K/V rows
    (all cached positions on full layers, the window on window layers)."""
    d, hd, heads, kv = config.hidden_size, config.head_dim, config.num_attention_heads, config.num_key_value_heads
    inter, top, layers = config.intermediate_size, config.experts_per_token, config.num_hidden_layers
    dense = d * hd * (heads + 2 * kv) + hd * (heads + 2 * kv) + hd * heads * d + d + d * config.num_experts + config.num_experts + 2 * d + heads
    experts = top * (2 * inter * d + 2 * inter + d * inter + d)
    full_kv = 2 * min(cached + 1, C5_CONTEXT) * kv * hd
    window_kv = 2 * min(cached + 1, config.sliding_window) * kv * hd
    kv_bytes = full_kv * (layers // 2) + window_kv * (layers - layers // 2)
    return 2 * (layers * (dense + experts) + kv_bytes + d * config.vocab_size + d)


def bench_c5(work: Path, steps: int, cpu: bool) -> dict:
    """C5: the GPT-OSS-20B-shaped bfloat16 model (24 layers, hidden 2880, 64/8 heads of 64, 32 experts
    top-4, vocabulary 201,088; weights N(0, 0.02) seed 2 drawn on the GPU). A 2048-token prefill through
    ``export_cached(m, 4096, 2048)`` (after one untimed prefill and a reset), a second prefill chunk that
    fills the 4096-position cache, then single-token steps through ``export_cached(m, 4096, 1)`` with the
    cache full. Device times run the plans on what their staging holds; ``Decoder`` times are end to end."""
    import shutil

    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd import Decoder
    from chroma_amd.models.cached import export_cached
    from chroma_amd.models.dev import make_gpt_oss_20b
    from chroma_amd.models.variants import gpt_oss_20b

    started = time.perf_counter()
    model = make_gpt_oss_20b(2, generator_device="cuda")
    torch.cuda.empty_cache()
    log(f"C5 weights drawn in {time.perf_counter() - started:.1f} s")
    programs = {}
    for name, steps_ in (("prefill", C5_PREFILL), ("decode", 1)):
        start = time.perf_counter()
        programs[name] = chroma_amd.compile(export_cached(model, C5_CONTEXT, steps_), work / f"c5_{name}")
        log(f"C5 {name} compiled and loaded in {time.perf_counter() - start:.1f} s ({programs[name].stats['launches']} launches)")
    del model
    tokens = torch.randint(0, VOCAB, (2 * C5_PREFILL + steps,), generator=torch.Generator().manual_seed(2)).numpy()
    result = {"workload": "GPT-OSS-20B-shaped bf16 MoE (24 layers, hidden 2880, 64/8 heads of 64, 32 experts top-4, vocab 201088, "
              "128-token windows on even layers), weights N(0,0.02) seed 2; 2048-token prefill from an empty 4096-position cache, "
              "then decode with all 4096 positions cached", "weight_bytes": programs["prefill"].stats["weight_bytes"],
              "launches": {name: program.stats["launches"] for name, program in programs.items()}}
    with Decoder(programs["prefill"], programs["decode"], sliding_window=gpt_oss_20b.sliding_window) as decoder:
        decoder.append(tokens[:C5_PREFILL])  # host staging's first touch and the mask-band cache
        decoder.reset()
        start = time.perf_counter()
        logits = decoder.append(tokens[:C5_PREFILL])
        result["prefill_decoder_ms"] = round((time.perf_counter() - start) * 1e3, 3)
        if not np.isfinite((logits.view(np.uint16).astype(np.uint32) << 16).view(np.float32)).all():
            raise RuntimeError("C5 prefill logits are not finite")
        prefill_ms = device_ms(programs["prefill"], 5, warmup=1)
        decoder.append(tokens[C5_PREFILL : 2 * C5_PREFILL])  # fills the cache: positions 0..4095
        samples = []
        for i in range(2 * C5_PREFILL, 2 * C5_PREFILL + steps):
            start = time.perf_counter()
            decoder.append(tokens[i : i + 1])
            samples.append((time.perf_counter() - start) * 1e3)
        result["decode_decoder_ms"] = round(statistics.median(samples), 3)
        result["decode_cache_on_device"] = decoder.stats["cache_on_device"]
        decode_ms = device_ms(programs["decode"], 20, warmup=2)
    flops = c5_live_flops(gpt_oss_20b, C5_PREFILL)
    decode_bytes = c5_decode_bytes(gpt_oss_20b, C5_CONTEXT)
    result.update({
        "prefill_device_ms": round(prefill_ms, 3),
        "prefill_live_flops": flops,
        "prefill_roofline": roofline(flops["total"], prefill_ms, bound="mfma"),
        "decode_device_ms": round(decode_ms, 4),
        "decode_algorithmic_bytes": decode_bytes,
        "decode_roofline": roofline(decode_bytes, decode_ms, traffic=read_traffic(C5_DECODE_TRAFFIC_FILE, "traffic_bytes_per_step")),
    })
    for name, program in programs.items():
        program.close()
        shutil.rmtree(work / f"c5_{name}", ignore_errors=True)
    if cpu:
        result["reduced_slice"] = c5_slice(work)
    return result


# Expert slot counts of one layer of the C5 bench prefill (2048 tokens x top-4 over 32 experts), sorted:
# the skewed routing the random-weight model actually produces in its later layers.
C5_SKEWED_COUNTS = (0, 0, 0, 2, 4, 4, 9, 12, 13, 21, 21, 38, 46, 59, 90, 109, 144, 147, 148, 159, 164, 176, 210, 220,
                    241, 269, 385, 427, 535, 1285, 1412, 1842)


def bench_experts(work: Path) -> dict:
    """The C5 expert products alone (up: [5760, 2880] per expert over the token rows; down: [2880, 2880] per
    expert over the slot rows; bf16, 2048 tokens x top-4 of 32) on the hip backend (routing launch plus
    the grouped matrix-core product), against the vendor library on the same work: one dense torch.mm of
    the same FLOPs (hipBLASLt; it reads one expert's weights instead of all 32), torch._grouped_mm over
    the experts' row groups, and one torch.mm per expert. Uniform routing (each token's 4 of 32 experts
    drawn at random) and C5's measured skew."""
    import numpy as np
    import torch

    import chroma_amd
    from tests.helpers import numpy_of

    experts, tokens, selected, inner = 32, 2048, 4, 2880

    class Up(torch.nn.Module):
        def __init__(self, w):
            super().__init__()
            self.w = torch.nn.Parameter(w, requires_grad=False)

        def forward(self, indices, x):
            return torch.einsum("beck,bk->bec", self.w[indices], x)

    class Down(Up):
        def forward(self, indices, x):
            return torch.einsum("beck,bek->bec", self.w[indices], x)

    def cuda_us(fn, runs: int = 20) -> float:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(runs):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / runs * 1e3

    generator = torch.Generator().manual_seed(0)
    uniform = torch.stack([torch.randperm(experts, generator=generator)[:selected] for _ in range(tokens)])
    order = torch.repeat_interleave(torch.arange(experts), torch.tensor(C5_SKEWED_COUNTS))
    skewed = torch.empty(tokens * selected, dtype=torch.int64)
    # expert runs laid over (slot, token) in token-fastest order, so a run of at most 2048 ids meets each token once
    skewed[(torch.arange(tokens * selected) % tokens) * selected + torch.arange(tokens * selected) // tokens] = order
    routings = {"uniform": uniform, "c5_skewed": skewed.reshape(tokens, selected)}
    result = {"workload": "C5 expert products, bf16, 2048 tokens x top-4 of 32 experts, K = 2880", "products": {}}
    for name, channels, per_slot in (("up", 5760, False), ("down", 2880, True)):
        w = (torch.randn(experts, channels, inner, generator=generator) * 0.02).to(torch.bfloat16)
        x = torch.randn(*((tokens, selected, inner) if per_slot else (tokens, inner)), generator=generator).to(torch.bfloat16)
        flops = 2 * tokens * selected * channels * inner
        entry = {"flops": flops, "hip": {}}
        for label, indices in routings.items():
            module = (Down if per_slot else Up)(w)
            with chroma_amd.compile(torch.export.export(module, (indices, x)), work / f"{name}_{label}") as program:
                program.native.upload([indices.numpy(), numpy_of(x)])
                us = device_ms(program, 20) * 1e3
            counts = np.bincount(indices.numpy().ravel(), minlength=experts)
            entry["hip"][label] = {"us": round(us, 1), "frac": round(flops / (us * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4),
                                   "slots_per_expert_min_max": [int(counts.min()), int(counts.max())]}
        wd = w.cuda()
        rows = tokens * selected
        xd = torch.randn(rows, inner, device="cuda", dtype=torch.bfloat16)
        dense = wd[0].contiguous()
        library = {"dense_mm_same_flops": cuda_us(lambda: torch.mm(xd, dense.t()))}
        offsets = torch.arange(1, experts + 1, device="cuda", dtype=torch.int32) * (rows // experts)
        if hasattr(torch, "_grouped_mm"):
            try:
                library["grouped_mm_uniform_groups"] = cuda_us(lambda: torch._grouped_mm(xd, wd.transpose(-2, -1), offs=offsets))
            except Exception as error:  # noqa: BLE001 - reported in the JSON line
                library["grouped_mm_uniform_groups"] = f"{type(error).__name__}: {str(error)[:120]}"
        parts = xd.view(experts, rows // experts, inner)
        library["mm_per_expert_uniform_groups"] = cuda_us(lambda: [torch.mm(parts[e], wd[e].t()) for e in range(experts)])
        entry["library_us"] = {key: round(value, 1) if isinstance(value, float) else value for key, value in library.items()}
        entry["library_frac"] = {key: round(flops / (value * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4)
                                 for key, value in library.items() if isinstance(value, float)}
        result["products"][name] = entry
        del wd, xd, dense
        torch.cuda.empty_cache()
    return result


def c5_slice(work: Path) -> dict:
    """C5 at full width on a reduced slice, hip beside the oracle: 2 layers (one sliding-window layer
    [window 16 at this context], one full layer), all 32 experts, a 64-position cache, a 32-token prefill
    chunk and 4 single-token steps, both through routing probes (``export_cached(..., routing=True)``).
    Reported: the oracle's time per call; the routing agreement over every (position, layer) decision
    with each flip and both runs' own gate-logit gaps (oracle/routing.py), and the same comparison of eager
    torch's bfloat16 forward (its own gate logits) with the oracle, the noise floor; per call, the logits row of its
    last position against the oracle's, with eager torch's bfloat16 forward against the oracle on the same
    row (the rounding noise floor), and whether the row depends on a flip. Every call is listed; the
    summary holds the calls that do not depend on a flip to the bfloat16 bar and names the others."""
    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd import Decoder
    from chroma_amd._src.dtypes import bf16_to_float32
    from chroma_amd.models.cached import export_cached
    from chroma_amd.models.dev import make_gpt_oss_20b
    from oracle import compile_cpu
    from oracle.routing import compare_routing, downstream_of

    def gathered(runs):
        runs = sorted(runs, key=lambda run: run[0])
        ids = np.concatenate([arrays[1][:, :count] for _, count, arrays in runs], axis=1)
        logits = np.concatenate([bf16_to_float32(arrays[0][:, :count]) for _, count, arrays in runs], axis=1)
        return ids, logits

    layers = 2
    model = make_gpt_oss_20b(2, num_hidden_layers=layers, num_experts=32, sliding_window=16)
    tokens = torch.randint(0, VOCAB, (36,), generator=torch.Generator().manual_seed(2))
    gates = []
    hooks = [block.mlp.gate.register_forward_hook(lambda module, args, out: gates.append(out.float().numpy())) for block in model.block]
    with torch.no_grad():
        eager = model(tokens).float().numpy()
    for hook in hooks:
        hook.remove()
    eager_logits = np.stack(gates)  # [layers, positions, experts]: eager torch's own bfloat16 gate logits
    eager_ids = torch.topk(torch.from_numpy(eager_logits), 4, dim=-1, sorted=True).indices.numpy()
    graphs = [export_cached(model, 64, 32, routing=True), export_cached(model, 64, 1, routing=True)]
    hip = [chroma_amd.compile(g, work / f"c5s_hip{i}") for i, g in enumerate(graphs)]
    cpu = [compile_cpu(g, work / f"c5s_cpu{i}") for i, g in enumerate(graphs)]
    tokens = tokens.numpy()
    times = {"hip": [], "cpu_oracle": []}
    rows = []
    hip_runs, cpu_runs = [], []
    with Decoder(*hip, sliding_window=16, extra_outputs=True) as decoder, Decoder(*cpu, sliding_window=16, extra_outputs=True) as reference:
        for start, end in ((0, 32), *((i, i + 1) for i in range(32, 36))):
            t0 = time.perf_counter()
            got = bf16_to_float32(decoder.append(tokens[start:end]))[-1]
            t1 = time.perf_counter()
            want = bf16_to_float32(reference.append(tokens[start:end]))[-1]
            t2 = time.perf_counter()
            times["hip"].append((t1 - t0) * 1e3)
            times["cpu_oracle"].append((t2 - t1) * 1e3)
            hip_runs += decoder.extras
            cpu_runs += reference.extras
            rows.append((end - 1, got, want))
    for program in (*hip, *cpu):
        program.close()
    oracle_routing = gathered(cpu_runs)
    routing = compare_routing(*gathered(hip_runs), *oracle_routing, bound_ulps=2.0)
    # the same comparison for eager torch's bfloat16 forward: how far another exact bfloat16 evaluation of
    # the model drifts from the oracle on the same decisions (the noise floor hip's flips sit against)
    eager_routing = compare_routing(eager_ids, eager_logits, *oracle_routing, bound_ulps=2.0)

    def flip_list(result, name):
        return [{"position": f["position"], "layer": f["layer"], f"{name}_ids": f["hip_ids"], "oracle_ids": f["ref_ids"],
                 f"gaps_ulps_{name}_oracle": [[p["hip_gap_ulps"], p["ref_gap_ulps"]] for p in f["pairs"]], "explained": f["explained"]}
                for f in result["flips"]]
    calls = []
    for position, got, want in rows:
        noise = eager[position]
        calls.append({"position": position, "downstream_of_flip": downstream_of(routing["flips"], position, layers),
                      "max_abs": round(float(np.abs(got - want).max()), 5),
                      "rel_norm": round(float(np.linalg.norm(got - want) / np.linalg.norm(want)), 5),
                      "argmax_equal": bool(got.argmax() == want.argmax()), "finite": bool(np.isfinite(got).all()),
                      "eager_vs_oracle_rel_norm": round(float(np.linalg.norm(noise - want) / np.linalg.norm(want)), 5)})
    held = [c for c in calls if not c["downstream_of_flip"]]
    summary = {
        "routing_agreement": routing["agreement"],
        "routing_decisions": f"{routing['matched']}/{routing['compared']} identical, {len(routing['tie_reorders'])} exact-tie reorders "
                             f"({routing['downstream']} downstream of a flip, {routing['downstream_matched']} of them agree)",
        "tie_reorders": [{"position": t["position"], "layer": t["layer"], "hip_ids": t["hip_ids"], "oracle_ids": t["ref_ids"],
                          "hip_lower_id_first": t["hip_lower_id_first"]} for t in routing["tie_reorders"]],
        "flips": flip_list(routing, "hip"),
        "unexplained_flips": routing["unexplained"],
        # flips beyond the bound whose gaps are still within how far eager torch's own gate logits drift
        # from the oracle's (another exact bfloat16 evaluation)
        "unexplained_within_eager_logit_drift": sum(
            1 for f in routing["flips"] if not f["explained"]
            and all(max(p["hip_gap_ulps"], p["ref_gap_ulps"]) <= eager_routing["logit_max_diff_ulps"] for p in f["pairs"])),
        "hip_ids_are_top4_of_own_logits": not routing["hip_selection_mismatches"],
        "gate_logits_max_diff_row_ulps": routing["logit_max_diff_ulps"],
        "flip_bound_ulps": routing["bound_ulps"],
        "eager_vs_oracle_routing": {"agreement": eager_routing["agreement"], "flips": flip_list(eager_routing, "eager"),
                                    "unexplained_flips": eager_routing["unexplained"],
                                    "gate_logits_max_diff_row_ulps": eager_routing["logit_max_diff_ulps"]},
        "calls_held": len(held), "calls_downstream_of_flip": [c["position"] for c in calls if c["downstream_of_flip"]],
        "held_rel_norm": max(c["rel_norm"] for c in held) if held else None,
        "held_max_abs": max(c["max_abs"] for c in held) if held else None,
        "held_argmax_equal": all(c["argmax_equal"] for c in held),
        "all_finite": all(c["finite"] for c in calls),
        "eager_vs_oracle_rel_norm": max(c["eager_vs_oracle_rel_norm"] for c in calls),
    }
    summary["held_within_bf16_bar"] = bool(held) and summary["held_rel_norm"] <= 2e-2 and summary["held_argmax_equal"] and summary["all_finite"]
    return {"slice": "2 layers (window 16, full), all 32 experts, hidden 2880, 64/8 heads, vocab 201088, cache 64, 32-token prefill + 4 steps, tokens seed 2",
            "hip_prefill_ms": round(times["hip"][0], 3), "cpu_prefill_ms": round(times["cpu_oracle"][0], 3),
            "hip_step_ms": round(statistics.median(times["hip"][1:]), 3), "cpu_step_ms": round(statistics.median(times["cpu_oracle"][1:]), 3),
            "parity": summary, "calls": calls}


# --------------------------------------------------------------------------------------------- counters
def counters(work: Path, which: str) -> None:
    """For rocprofv3 --pmc: the named plan replayed three times, then three launches of a plain copy kernel of
    known size (``x * 1.0`` over a [16384, 8192] fp32 input: 512 MiB read, 512 MiB written), which calibrates
    FETCH_SIZE / WRITE_SIZE on the same GPU. ``c2``: the C2 kernel. ``c5``: the C5 decode plan with all 4096
    cache positions valid (two 2048-token prefills fill the cache first). ``c5prefill``: the C5 2048-token
    prefill plan (for the matrix-core counters). ``rows``: every row-reduction case of the rows leg in turn.
    ``c1``, ``dev``, ``decode``: the C1 block, the C3 forward and the C4 decode step (after an 8-token prefill
    and one step). Each plan's kernel names are logged, in launch order, before it runs."""
    import torch

    import chroma_amd
    from chroma_amd.models.blocks import BandwidthGraph, Copy, bandwidth_inputs

    def replay(program, directory: Path, label: str) -> None:
        log(f"{label}: {program.stats['launches']} launch(es) x3: {' '.join(plan_kernels(directory))}")
        program.native.execute(3)

    x, y = bandwidth_inputs()
    if which == "c2":
        program = chroma_amd.compile(torch.export.export(BandwidthGraph(), (x, y)), work / "c2")
        program.native.upload([x.numpy(), y.numpy()])
        replay(program, work / "c2", "c2")
        program.close()
    elif which == "c5":
        c5_decode_counters(work)
    elif which == "c5prefill":
        c5_prefill_counters(work)
    elif which == "rows":
        for kind, rows, width in ROW_CASES:
            module, data = row_case_module(kind, rows, width)
            directory = work / f"{kind}_{rows}_{width}"
            with chroma_amd.compile(torch.export.export(module, (data,)), directory) as program:
                program.native.upload([data.numpy()])
                replay(program, directory, f"{kind} [{rows},{width}]")
    elif which == "c1":
        from chroma_amd.models.blocks import mlp_block, mlp_inputs

        module, (data,) = mlp_block(), mlp_inputs()
        with chroma_amd.compile(torch.export.export(module, (data,)), work / "c1") as program:
            program.native.upload([data.numpy()])
            replay(program, work / "c1", "c1")
    elif which == "dev":
        from chroma_amd.models.dev import make_dev_model

        tokens = torch.randint(0, VOCAB, (8,), generator=torch.Generator().manual_seed(0))
        with chroma_amd.compile(torch.export.export(make_dev_model(0), (tokens,)), work / "dev") as program:
            program.native.upload([tokens.numpy()])
            replay(program, work / "dev", "dev")
    elif which == "decode":
        from chroma_amd import Decoder
        from chroma_amd.models.cached import export_cached
        from chroma_amd.models.dev import make_dev_model

        model = make_dev_model(0)
        prefill = chroma_amd.compile(export_cached(model, 256, 256), work / "prefill")
        decode = chroma_amd.compile(export_cached(model, 256, 1), work / "decode")
        tokens = torch.randint(0, VOCAB, (9,), generator=torch.Generator().manual_seed(0)).numpy()
        with Decoder(prefill, decode) as decoder:
            decoder.append(tokens[:8])
            decoder.append(tokens[8:])
            replay(decode, work / "decode", "decode")
    program = chroma_amd.compile(torch.export.export(Copy(), (x,)), work / "copy")
    program.native.upload([x.numpy()])
    replay(program, work / "copy", "copy")
    program.close()


def c5_prefill_counters(work: Path) -> None:
    """The C5 2048-token prefill plan replayed three times (after one prefill through ``Decoder``)."""
    import torch

    import chroma_amd
    from chroma_amd import Decoder
    from chroma_amd.models.cached import export_cached
    from chroma_amd.models.dev import make_gpt_oss_20b
    from chroma_amd.models.variants import gpt_oss_20b

    model = make_gpt_oss_20b(2, generator_device="cuda")
    torch.cuda.empty_cache()
    prefill = chroma_amd.compile(export_cached(model, C5_CONTEXT, C5_PREFILL), work / "c5_prefill")
    decode = chroma_amd.compile(export_cached(model, C5_CONTEXT, 1), work / "c5_decode")
    del model
    tokens = torch.randint(0, VOCAB, (C5_PREFILL,), generator=torch.Generator().manual_seed(2)).numpy()
    with Decoder(prefill, decode, sliding_window=gpt_oss_20b.sliding_window) as decoder:
        decoder.append(tokens)
        torch.cuda.synchronize()
        log(f"C5 prefill: {prefill.stats['launches']} launch(es) x3: {' '.join(plan_kernels(work / 'c5_prefill'))}")
        prefill.native.execute(3)


def c5_decode_counters(work: Path) -> None:
    """The C5 decode plan replayed three times on a full cache (the setup of ``bench_c5``)."""
    import torch

    import chroma_amd
    from chroma_amd import Decoder
    from chroma_amd.models.cached import export_cached
    from chroma_amd.models.dev import make_gpt_oss_20b
    from chroma_amd.models.variants import gpt_oss_20b

    model = make_gpt_oss_20b(2, generator_device="cuda")
    torch.cuda.empty_cache()
    prefill = chroma_amd.compile(export_cached(model, C5_CONTEXT, C5_PREFILL), work / "c5_prefill")
    decode = chroma_amd.compile(export_cached(model, C5_CONTEXT, 1), work / "c5_decode")
    del model
    tokens = torch.randint(0, VOCAB, (2 * C5_PREFILL + 1,), generator=torch.Generator().manual_seed(2)).numpy()
    with Decoder(prefill, decode, sliding_window=gpt_oss_20b.sliding_window) as decoder:
        decoder.append(tokens[:C5_PREFILL])
        decoder.append(tokens[C5_PREFILL : 2 * C5_PREFILL])
        decoder.append(tokens[2 * C5_PREFILL :])
        torch.cuda.synchronize()
        decode.native.execute(3)
        log(f"C5 decode: ran {decode.stats['launches']} launch(es) x3")
    prefill.close()
    decode.close()


def run_leg(name: str, leg, work: Path):
    """One secondary measurement in a directory of its own, removed afterwards (the C5 artifacts alone hold
    42 GB of weights); a failure is recorded in the line instead of losing the headline."""
    import shutil
    import traceback

    directory = work / name
    directory.mkdir()
    start = time.perf_counter()
    try:
        result = leg(directory)
        log(f"{name} done in {time.perf_counter() - start:.1f} s")
        return result
    except Exception as error:  # noqa: BLE001 - reported in the JSON line
        traceback.print_exc()
        return {"error": f"{type(error).__name__}: {error}"}
    finally:
        shutil.rmtree(directory, ignore_errors=True)


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-extras", action="store_true", help="only the C2 headline (and its CPU baseline)")
    parser.add_argument("--no-cpu", action="store_true", help="skip every oracle (CPU) measurement")
    parser.add_argument("--no-c5", action="store_true", help="skip the GPT-OSS-20B-shaped model (about two minutes: 42 GB of weights)")
    parser.add_argument("--counters", nargs="?", const="c2", choices=["c2", "c5", "c5prefill", "rows", "c1", "dev", "decode"],
                        help="only replay one plan (C2 kernel by default; c5 = the C5 decode step) and a copy kernel, for rocprofv3 --pmc")
    parser.add_argument("--only", choices=["c1", "rows", "dev", "decode", "c5", "experts"],
                        help="measure one leg and print it (experts: the C5 expert products against the vendor library)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the hip backend is single-device (every GPU box here has one GPU)", file=sys.stderr)
        sys.exit(2)
    cpu = not args.no_cpu

    with tempfile.TemporaryDirectory(prefix="chroma-bench-") as directory:
        work = Path(directory)
        if args.counters:
            counters(work, args.counters)
            return
        if args.only:
            legs = {"c1": lambda: bench_c1(work, cpu), "rows": lambda: bench_rows(work, cpu), "dev": lambda: bench_dev(work, cpu),
                    "decode": lambda: bench_decode(work, 32, cpu), "c5": lambda: bench_c5(work, 16, cpu),
                    "experts": lambda: bench_experts(work)}
            print(json.dumps({args.only: legs[args.only]()}), flush=True)
            return
        c2 = bench_c2(args, work)
        log(f"C2 {c2['value']:.1f} GB/s wall, kernel {c2['kernel_ms']:.4f} ms ({c2['roofline']['achieved']:.1f} GB/s)")
        line = {
            "metric": METRIC,
            "value": round(c2["value"], 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(c2["ms_per_step"], 5),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "f32",
            "data": "synthetic",
            "config": {
                "workload": "C2 bandwidth graph: softmax(tanh(x*0.5+y)*sigmoid(y)-exp(clamp(x,-8,8))*1e-3, -1), fp32 x,y~U(-4,4) [16384,8192] seed 1, inputs resident in HBM",
                "algorithmic_bytes_per_step": C2_BYTES,
                "launches_per_step": c2["stats"]["launches"],
                "end_to_end_ms_with_pcie": c2["end_to_end_ms"]["median_ms"],
            },
            "roofline": c2["roofline"],
            "cpu_baseline": cpu_c2(work) if cpu else None,
        }
        line["host"] = dict(host_info(), gpu=c2["device"])
        if not args.no_extras:
            legs = [("hbm_copy", lambda d: bench_copy(d)), ("rows", lambda d: bench_rows(d, cpu)), ("c1", lambda d: bench_c1(d, cpu)),
                    ("dev_forward", lambda d: bench_dev(d, cpu)), ("decode", lambda d: bench_decode(d, 32, cpu))]
            if not args.no_c5:
                legs.append(("c5", lambda d: bench_c5(d, 16, cpu)))
            for name, leg in legs:
                line[name] = run_leg(name, leg, work)
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
