"""Benchmark of the hip backend on one MI355X.

Headline (``value``): the fused-kernel HBM throughput of BASELINE config C2 - the fp32 bandwidth graph
``softmax(tanh(x*0.5+y)*sigmoid(y) - exp(clamp(x,-8,8))*1e-3, -1)`` over x, y in U(-4, 4) [16384, 8192]
(generator seed 1, x then y) compiled with ``chroma_amd.compile(..., backend="hip")``. One step is one
execution of the compiled program on inputs already resident in HBM; GB/s counts the algorithmic bytes
(read x, read y, write the output: 3 x 16384 x 8192 x 4 = 1,610,612,736 B per step).

Beside it the same JSON line reports:

* ``roofline``: the dominant kernel's algorithmic bytes over its average duration from hipEvents recorded
  on the runtime's own stream around the timed launches, against MI355X's 8 TB/s; ``traffic`` comes from
  the committed rocprofv3 FETCH_SIZE/WRITE_SIZE measurement (profiles/) when present;
* ``cpu_baseline``: the CPU restatement of Chroma's CPU backend (oracle/, single thread, BLAS pinned to one
  thread) timed on this host on a bounded sample of the same graph;
* ``dev_forward`` / ``decode``: the dev MoE model's 8-token forward and its 256-position KV-cached decode
  step (BASELINE configs C3 and C4), end-to-end from host arrays to host arrays, with the oracle's times.
"""

from __future__ import annotations

import argparse
import json
import os
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
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = ROOT / "profiles" / "c2_fused_softmax_traffic.txt"


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def c2_module():
    import torch

    class BandwidthGraph(torch.nn.Module):
        def forward(self, x, y):
            z = torch.tanh(x * 0.5 + y) * torch.sigmoid(y) - torch.exp(torch.clamp(x, -8, 8)) * 1e-3
            return torch.softmax(z, -1)

    return BandwidthGraph()


def c2_inputs(rows: int = C2_SHAPE[0], cols: int = C2_SHAPE[1]):
    import torch

    generator = torch.Generator().manual_seed(1)
    x = torch.rand(rows, cols, generator=generator) * 8 - 4
    y = torch.rand(rows, cols, generator=generator) * 8 - 4
    return x, y


def read_traffic():
    """HBM bytes per C2 launch from the committed rocprofv3 counter summary, or None."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return int(float(line.split()[-1]))
    return None


def bench_c2(args, work: Path) -> dict:
    import numpy as np
    import torch

    import chroma_amd

    x, y = c2_inputs()
    exported = torch.export.export(c2_module(), (x, y))
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
    sums = output[:: 1024].sum(axis=1)
    if not np.allclose(sums, 1.0, rtol=1e-4):
        raise RuntimeError(f"C2 rows do not sum to 1: {sums[:4]}")
    kernel_ms = event_ms / args.steps
    achieved = C2_BYTES / (kernel_ms * 1e-3) / 1e9
    traffic = read_traffic()
    program.close()
    return {
        "value": C2_BYTES * args.steps / wall / 1e9,
        "ms_per_step": wall / args.steps * 1e3,
        "kernel_ms": kernel_ms,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "stats": program.stats,
    }


def cpu_c2(work: Path) -> dict:
    """The oracle on a bounded sample of C2 (the first rows), one thread."""
    import numpy as np
    import torch

    from oracle import compile_cpu

    rows = 2048
    x, y = c2_inputs()
    x, y = x[:rows].contiguous(), y[:rows].contiguous()
    program = compile_cpu(torch.export.export(c2_module(), (x, y)), work / "c2_cpu")
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
    return {
        "value": round(sample_bytes / seconds / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"C2 graph on the first {rows} of 16384 rows ([{rows},8192] x2 fp32), median of {len(times)} runs, "
        f"{seconds * 1e3:.1f} ms each; oracle = CPU restatement of Chroma's CPU backend, -O3 -ffp-contract=off, 1 thread",
    }


def timed(call, warmup: int, runs: int) -> dict:
    for _ in range(warmup):
        call()
    samples = []
    for _ in range(runs):
        start = time.perf_counter()
        call()
        samples.append((time.perf_counter() - start) * 1e3)
    return {"median_ms": round(statistics.median(samples), 4), "p10_ms": round(sorted(samples)[len(samples) // 10], 4), "runs": runs}


def bench_dev(work: Path, runs: int) -> dict:
    """C3: the dev model's 8-token fp32 forward, host arrays in and out, and the oracle beside it."""
    import numpy as np
    import torch

    import chroma_amd
    from chroma_amd.models.dev import make_dev_model, weights_digest
    from oracle import compile_cpu

    model = make_dev_model(0)
    tokens = torch.randint(0, 201088, (8,), generator=torch.Generator().manual_seed(0))
    exported = torch.export.export(model, (tokens,))
    log("compiling the dev model for hip and the oracle")
    program = chroma_amd.compile(exported, work / "dev")
    oracle = compile_cpu(exported, work / "dev_cpu")
    array = tokens.numpy()
    got, want = program(array), oracle(array)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    argmax_equal = bool((got.argmax(-1) == want.argmax(-1)).all())
    out = program(array)  # the reference's out= method reuses an earlier result (scripts/benchmark.py:207-208)
    pageable = np.empty_like(got)
    result = {
        "workload": "dev MoE model (12 layers, 59,079,408 params, vocab 201088), 8-token fp32 forward, batch 1, tokens ~U[0,201088) seed 0",
        "weights_sha256": weights_digest(model),
        "hip_fresh": timed(lambda: program(array), 10, runs),
        "hip_reuse": timed(lambda: program(array, out=out), 10, runs),
        "hip_reuse_pageable_out": timed(lambda: program(array, out=pageable), 10, runs),
        "cpu_oracle": timed(lambda: oracle(array), 2, max(5, runs // 10)),
        "argmax_equal": argmax_equal,
        "launches": program.stats["launches"],
    }
    native = program.native
    native.upload([array])
    native.execute(5)
    result["hip_device_only_ms"] = round(native.execute(runs, timed=True) / runs, 4)
    program.close()
    oracle.close()
    return result


def bench_decode(work: Path, steps: int) -> dict:
    """C4: dev model KV-cached decode at a 256-position cache through ``Decoder`` (host mask and cache
    work included), plus the padded uncached 256-token graph, with the oracle's times."""
    import numpy as np

    import chroma_amd
    from chroma_amd import Decoder
    from chroma_amd.models.cached import export_cached, export_uncached
    from chroma_amd.models.dev import make_dev_model
    from oracle import compile_cpu

    model = make_dev_model(0)
    graphs = {"prefill": export_cached(model, 256, 256), "decode": export_cached(model, 256, 1), "full": export_uncached(model, 256)}
    log("compiling the decode graphs for hip and the oracle")
    hip = {name: chroma_amd.compile(graph, work / f"hip_{name}") for name, graph in graphs.items()}
    cpu = {name: compile_cpu(graph, work / f"cpu_{name}") for name, graph in graphs.items()}
    tokens = ((np.arange(8 + steps, dtype=np.int64) * 7919 + 17) % 201088).astype(np.int64)
    results = {}
    for name, programs in (("hip", hip), ("cpu_oracle", cpu)):
        decoder = Decoder(programs["prefill"], programs["decode"])
        decoder.append(tokens[:8])
        samples = []
        count = steps if name == "hip" else min(steps, 8)
        for i in range(8, 8 + count):
            start = time.perf_counter()
            decoder.append(tokens[i : i + 1])
            samples.append((time.perf_counter() - start) * 1e3)
        greedy = None
        if name == "hip":
            # the same steps through Decoder.greedy: the logits stay on the device and a selection program
            # returns the chosen id (8 bytes down instead of the 804 KB row)
            decoder.reset()
            decoder.append(tokens[:8])
            decoder.greedy(tokens[8:9])  # compiles the selection program
            greedy = []
            for i in range(9, 8 + count):
                start = time.perf_counter()
                decoder.greedy(tokens[i : i + 1])
                greedy.append((time.perf_counter() - start) * 1e3)
            decoder.close()
        padded = np.zeros(256, dtype=np.int64)
        padded[:16] = tokens[:16]
        last = np.array([15], dtype=np.int64)
        full = programs["full"]
        results[name] = {
            "decode_step": {"median_ms": round(statistics.median(samples), 4), "steps": count},
            "uncached_256": timed(lambda: full(padded, last), 2, 10 if name == "hip" else 3),
            "uncached_logits": full(padded, last),
        }
        if greedy:
            results[name]["decode_step_greedy"] = {"median_ms": round(statistics.median(greedy), 4), "steps": len(greedy)}
    np.testing.assert_allclose(results["hip"]["uncached_logits"], results["cpu_oracle"]["uncached_logits"], rtol=1e-4, atol=1e-5)
    for entry in results.values():
        entry.pop("uncached_logits")
    for program in (*hip.values(), *cpu.values()):
        program.close()
    results["workload"] = "dev model, Decoder(export_cached(m,256,256), export_cached(m,256,1)), prefill 8 tokens then single-token steps; padded export_uncached(m,256)"
    return results


C5_CONTEXT, C5_PREFILL = 4096, 2048


def c5_flops(config, tokens: int, context: int) -> dict:
    """Multiply-add work (2 flops each) of one pass of ``export_cached(m, context, tokens)``, per kind of
    product, as the graph computes it (every score over the whole padded cache; one row unembedded)."""
    d, hd, heads, kv = config.hidden_size, config.head_dim, config.num_attention_heads, config.num_key_value_heads
    inter, top, layers = config.intermediate_size, config.experts_per_token, config.num_hidden_layers
    keys = context + tokens
    per_layer = {
        "qkv": 2 * tokens * d * hd * (heads + 2 * kv),
        "out": 2 * tokens * hd * heads * d,
        "router": 2 * tokens * d * config.num_experts,
        "experts_up": 2 * tokens * top * 2 * inter * d,
        "experts_down": 2 * tokens * top * d * inter,
        "scores": 2 * heads * tokens * keys * hd,
        "attend": 2 * heads * tokens * keys * hd,
    }
    flops = {name: value * layers for name, value in per_layer.items()}
    flops["unembedding"] = 2 * d * config.vocab_size
    flops["total"] = sum(flops.values())
    return flops


def c5_decode_bytes(config, context: int) -> int:
    """HBM bytes one decode step must read at least: every dense weight, the four selected experts of
    every layer, the K/V cache, the unembedding, in bfloat16 (norm scales and biases ignored)."""
    d, hd, heads, kv = config.hidden_size, config.head_dim, config.num_attention_heads, config.num_key_value_heads
    inter, top = config.intermediate_size, config.experts_per_token
    per_layer = d * hd * (heads + 2 * kv) + hd * heads * d + d * config.num_experts + top * (2 * inter * d + d * inter)
    cache = 2 * context * kv * hd
    return 2 * (config.num_hidden_layers * (per_layer + cache) + d * config.vocab_size)


def bench_c5(work: Path, steps: int) -> dict:
    """C5: the GPT-OSS-20B-shaped bfloat16 model (24 layers, hidden 2880, 64/8 heads of 64, 32 experts
    top-4, vocabulary 201,088; weights N(0, 0.02) seed 2 drawn on the GPU), a 2048-token prefill through
    ``export_cached(m, 4096, 2048)`` and single-token steps through ``export_cached(m, 4096, 1)``. Device
    times run on device-resident inputs; the ``Decoder`` times are end to end (host cache and masks)."""
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
    tokens = torch.randint(0, 201088, (C5_PREFILL + steps,), generator=torch.Generator().manual_seed(2)).numpy()
    result = {"workload": "GPT-OSS-20B-shaped bf16 MoE (24 layers, hidden 2880, 64/8 heads of 64, 32 experts top-4, vocab 201088), "
              "weights N(0,0.02) seed 2; 2048-token prefill (timed after one untimed prefill and a reset) then decode, cache 4096 positions",
              "weight_bytes": programs["prefill"].stats["weight_bytes"]}
    flops = c5_flops(gpt_oss_20b, C5_PREFILL, C5_CONTEXT)
    with Decoder(programs["prefill"], programs["decode"], sliding_window=gpt_oss_20b.sliding_window) as decoder:
        # one untimed prefill first: the host staging's first touch and the decoder's mask-band cache
        decoder.append(tokens[:C5_PREFILL])
        decoder.reset()
        start = time.perf_counter()
        logits = decoder.append(tokens[:C5_PREFILL])
        result["prefill_decoder_ms"] = round((time.perf_counter() - start) * 1e3, 3)
        if not np.isfinite((logits.view(np.uint16).astype(np.uint32) << 16).view(np.float32)).all():
            raise RuntimeError("C5 prefill logits are not finite")
        samples = []
        for i in range(C5_PREFILL, C5_PREFILL + steps):
            start = time.perf_counter()
            decoder.append(tokens[i : i + 1])
            samples.append((time.perf_counter() - start) * 1e3)
        result["decode_decoder_ms"] = round(statistics.median(samples), 3)
        result["decode_cache_on_device"] = decoder.stats["cache_on_device"]
        # Device-only times: the plans re-run on what their staging regions hold after the Decoder calls.
        for name, runs in (("prefill", 5), ("decode", 20)):
            native = programs[name].native
            native.execute(2)
            device_ms = native.execute(runs, timed=True) / runs
            result[f"{name}_device_ms"] = round(device_ms, 4)
    result["prefill_flops"] = flops["total"]
    result["prefill_tflops"] = round(flops["total"] / (result["prefill_device_ms"] * 1e-3) / 1e12, 1)
    result["prefill_mfma_frac"] = round(result["prefill_tflops"] / BF16_MFMA_PEAK_TFLOPS, 4)
    decode_bytes = c5_decode_bytes(gpt_oss_20b, C5_CONTEXT)
    result["decode_algorithmic_bytes"] = decode_bytes
    result["decode_gbs"] = round(decode_bytes / (result["decode_device_ms"] * 1e-3) / 1e9, 1)
    result["decode_hbm_frac"] = round(result["decode_gbs"] / HBM_PEAK_GBS, 4)
    return result


def counters(work: Path) -> None:
    """For rocprofv3 --pmc: three launches of the C2 kernel and of a plain copy kernel of known size
    (``x * 1.0`` over the same [16384, 8192] fp32 input: 512 MiB read, 512 MiB written), which calibrates
    FETCH_SIZE / WRITE_SIZE."""
    import torch

    import chroma_amd

    x, y = c2_inputs()
    programs = [
        (chroma_amd.compile(torch.export.export(c2_module(), (x, y)), work / "c2"), [x.numpy(), y.numpy()]),
        (chroma_amd.compile(torch.export.export(_copy_module(), (x,)), work / "copy"), [x.numpy()]),
    ]
    for program, arrays in programs:
        program.native.upload(arrays)
        program.native.execute(3)
        log(f"ran {program.stats['launches']} launch(es) x3")
        program.close()


def _copy_module():
    import torch

    class Copy(torch.nn.Module):
        def forward(self, x):
            return x * 1.0

    return Copy()


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-extras", action="store_true", help="skip the dev-model forward and decode measurements")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--counters", action="store_true", help="only run the C2 and copy kernels (for rocprofv3 --pmc)")
    parser.add_argument("--c5", action="store_true", help="also measure the GPT-OSS-20B-shaped bf16 model (minutes: 42 GB of weights)")
    parser.add_argument("--c5-only", action="store_true", help="only measure the GPT-OSS-20B-shaped model")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the hip backend is single-device (every GPU box here has one GPU)", file=sys.stderr)
        sys.exit(2)

    with tempfile.TemporaryDirectory(prefix="chroma-bench-") as directory:
        work = Path(directory)
        if args.counters:
            counters(work)
            return
        if args.c5_only:
            print(json.dumps({"c5": bench_c5(work, 16)}), flush=True)
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
            },
            "roofline": c2["roofline"],
            "cpu_baseline": None if args.no_cpu else cpu_c2(work),
        }
        if not args.no_extras:
            line["dev_forward"] = bench_dev(work, 100)
            log(f"dev forward {line['dev_forward']['hip_fresh']['median_ms']} ms (oracle {line['dev_forward']['cpu_oracle']['median_ms']} ms)")
            line["decode"] = bench_decode(work, 32)
            log(f"decode step {line['decode']['hip']['decode_step']['median_ms']} ms")
        if args.c5:
            line["c5"] = bench_c5(work, 16)
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
