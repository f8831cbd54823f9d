"""Decode throughput of the MI355X Mesh GPT generate path.

Workload ("mid"): vocabulary 256, width 512, 8 heads x 64,
6 blocks, butterfly meshes of depth 9, context 1024, batch 32, 64-token
uniform-random prompts, temperature 1.0 with per-sequence seeds 7+b; seeded
reference initialisation (seed 7).  A step is one decode step of the whole
batch (32 tokens).  Prompts are prefilled untimed; the timed region is K decode
steps starting right after the prompt (K = 512 is the full config-3 run), with
every input already resident in HBM.

The K steps run as one launch of the persistent decode kernel, so the timed
region is that kernel: HIP events recorded on the model's stream right
before and after the launch give its duration, and the roofline divides the
steps' algorithmic HBM bytes (KV-cache reads and appends, mesh weights, tied
head table, token ids) by it.  Prints one JSON line with that roofline, the
batch-1 (config 1) figure and the CPU baseline (the f64 oracle on one core, a
bounded sample of the workload).
"""
import argparse
import ctypes
import glob
import json
import os
import platform
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import grokking_abmod_amd as G  # noqa: E402

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
METRIC = "decode tokens/sec @1 GPU (batch 1 and 32) + % of HBM roofline per decode step"


class Hip:
    """hipEvent timing on a given stream through libamdhip64."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipDeviceSynchronize.argtypes = []

    def event(self):
        e = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, event, stream):
        assert self.lib.hipEventRecord(event, stream) == 0

    def elapsed_ms(self, start, stop):
        assert self.lib.hipEventSynchronize(stop) == 0
        ms = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), start, stop) == 0
        return ms.value

    def synchronize(self):
        assert self.lib.hipDeviceSynchronize() == 0


def prompts_for(config, batch, length, seed=7):
    """Uniform token ids from Random::new(seed).index(V), sequence b after b-1."""
    state = [seed]

    def next_u64():
        state[0] = (state[0] + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = state[0]
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    bound = config.vocab_size
    threshold = ((1 << 64) - bound) % bound
    out = np.empty((batch, length), dtype=np.uint32)
    for b in range(batch):
        for i in range(length):
            while True:
                bits = next_u64()
                if bits >= threshold:
                    out[b, i] = bits % bound
                    break
    return out


def step_bytes(config, batch, position):
    """Algorithmic HBM bytes of a whole decode step (all layers): KV reads and
    appends, mesh weights, the tied head table and the token ids."""
    w, layers = config.width, config.layers
    meshes = 4 * config.attention_mesh_depth + config.ffn_mesh_depth
    return (batch * layers * 2 * w * 4 * (position + 1) + batch * layers * 2 * w * 4
            + 8 * w * layers * meshes + 4 * config.vocab_size * w + 4 * batch)


def run_decode(hip, model, prompts, steps, temperature, seed):
    """Prefill (untimed) then `steps` timed decode steps (one persistent launch
    when the model supports it); returns (event ms, wall ms)."""
    model.prefill(prompts, temperature, seed, reserve=prompts.shape[1] + 1 + steps)
    hip.synchronize()
    stream = model.stream()
    start, stop = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(start, stream)
    model.decode(steps)
    hip.record(stop, stream)
    hip.synchronize()
    wall = (time.perf_counter() - t0) * 1000.0
    return hip.elapsed_ms(start, stop), wall


def cpu_baseline(config, prompts, steps, temperature, budget_s):
    """The f64 oracle's KV-cached decode on one host core over whole sequences
    of the workload (prompt + all decode steps), until budget_s is spent."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    o = O.config(**{k: v for k, v in config.as_dict().items() if k != "long_context"})
    params = O.initialize(o, 7)
    tokens = 0
    seconds = 0.0
    done = 0
    for b in range(prompts.shape[0]):
        t0 = time.perf_counter()
        O.generate(o, params, prompts[b], 1, temperature, 7 + b, cached=True)
        t1 = time.perf_counter()
        O.generate(o, params, prompts[b], 1 + steps, temperature, 7 + b, cached=True)
        t2 = time.perf_counter()
        seconds += (t2 - t1) - (t1 - t0)
        tokens += steps
        done += 1
        if t2 - t0 + seconds > budget_s:
            break
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(tokens / seconds, 2),
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{done} of {prompts.shape[0]} sequences, each its {prompts.shape[1]}-token prompt "
                  f"then {steps} decode steps; decode time only; f64 KV-cached oracle; {cpu}",
    }


KERNEL = "persistent_decode_kernel"


def pmc_traffic(args, config, batch):
    """HBM bytes of the persistent decode launch of the timed steps, from two
    rocprofv3 --pmc runs of a child process (FETCH_SIZE, then WRITE_SIZE), each
    scaled by the same counter on a plain copy kernel of known size.  Returns
    None when unavailable."""
    rocprof = "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rocprof):
        return None
    import csv

    def collect(counter):
        # rocprofv3 may exit with a segmentation fault after the program ends
        # (cooperative launches); the counter file is complete by then.
        out = tempfile.mkdtemp(prefix="mg_pmc_")
        cmd = ["timeout", "-s", "KILL", "90", rocprof, "--pmc", counter, "-d", out, "-o", "pmc",
               "--output-format", "csv", "--", sys.executable, os.path.abspath(__file__), "--probe",
               "--steps", str(args.steps), "--prompt", str(args.prompt), "--batch", str(batch)]
        res = subprocess.run(cmd, cwd="/tmp", capture_output=True, text=True)
        hits, copy = [], []
        for path in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for row in csv.DictReader(f):
                    name = row.get("Kernel_Name", "")
                    value = float(row.get("Counter_Value", "nan"))
                    if KERNEL in name:
                        hits.append(value)
                    elif "calibration_copy" in name:
                        copy.append(value)
        if not hits or not copy:
            sys.stderr.write(f"pmc {counter}: kernel rows {len(hits)}, copy rows {len(copy)} "
                             f"(rc={res.returncode})\n{res.stderr[-1500:]}\n")
        return hits, copy

    per_counter = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        hits, copy = collect(counter)
        if not hits or not copy:
            hits, copy = collect(counter)
        if not hits or not copy:
            return None
        copy_kib = PROBE_COPY_BYTES / 1024.0
        factor = copy_kib / float(np.mean(copy))
        per_counter[counter] = float(np.mean(hits)) * factor * 1024.0
        per_counter[counter + "_factor"] = factor
    return per_counter


PROBE_COPY_BYTES = 256 << 20


def probe(args):
    """Child process under rocprofv3 --pmc: the timed region's decode steps (same
    positions, one persistent launch) and one plain copy kernel of known size
    for calibration."""
    config = G.named_config("mid")
    prompts = prompts_for(config, args.batch, args.prompt)
    with G.MeshGpt(0, config, 7, max_batch=args.batch) as model:
        model.prefill(prompts, 1.0, 7, reserve=args.prompt + 1 + args.steps)
        model.decode(args.steps)
    G.calibration_copy(PROBE_COPY_BYTES)


def batch1_figure(hip, steps=128):
    """batch 1, 16-token prompt, greedy decode 128 tokens."""
    config = G.named_config("tiny")
    prompts = prompts_for(config, 1, 16)
    with G.MeshGpt(0, config, 7) as model:
        run_decode(hip, model, prompts, steps, 0.0, 7)  # warm-up
        ms, _ = run_decode(hip, model, prompts, steps, 0.0, 7)
    return {"workload": "config 1 (tiny): V64 W128 H4x32 L2 butterfly depth 7, ctx 256, batch 1, "
                        "16-token prompt, 128 greedy decode steps",
            "tokens_per_s": round(steps / (ms / 1000.0), 1), "us_per_token": round(1000.0 * ms / steps, 2)}


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=512)
    parser.add_argument("--warmup", type=int, default=16)
    parser.add_argument("--batch", type=int, default=32)
    parser.add_argument("--prompt", type=int, default=64)
    parser.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-pmc", action="store_true")
    parser.add_argument("--probe", action="store_true", help=argparse.SUPPRESS)
    args = parser.parse_args()

    if args.probe:
        probe(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "decode would shard by sequence with no per-step exchange between GPUs.", file=sys.stderr)
        sys.exit(2)

    config = G.named_config("mid")
    if args.prompt + args.steps > config.context or args.prompt + args.warmup > config.context:
        sys.exit(f"prompt + steps must stay within the context ({config.context})")
    # The counter runs go first, while this process has not touched the GPU:
    # the profiled child is then the only process on it.
    traffic = None
    pmc = None
    if not args.no_pmc:
        try:
            pmc = pmc_traffic(args, config, args.batch)
        except Exception as exc:  # counters are optional evidence, never the result
            sys.stderr.write(f"pmc collection failed: {exc}\n")
            pmc = None
        if pmc:
            traffic = round(pmc["FETCH_SIZE"] + pmc["WRITE_SIZE"])
    temperature = 1.0
    prompts = prompts_for(config, args.batch, args.prompt)
    hip = Hip()
    with G.MeshGpt(0, config, 7, max_batch=args.batch) as model:
        # Warm-up: a full prefill and W decode steps.
        if args.warmup:
            model.prefill(prompts, temperature, 7, reserve=args.prompt + 1 + max(args.steps, args.warmup))
            model.decode(args.warmup)
            hip.synchronize()
        ms, wall_ms = run_decode(hip, model, prompts, args.steps, temperature, 7)

    positions = args.prompt + np.arange(args.steps)
    total_bytes = float(sum(step_bytes(config, args.batch, p) for p in positions))
    gbps = total_bytes / (ms / 1000.0) / 1e9

    result = {
        "metric": METRIC,
        "value": round(args.batch * args.steps / (ms / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "config 3 (mid): V256 W512 H8x64 L6 butterfly depth 9, ctx 1024, batch 32, "
                        "64-token uniform-random prompts, T=1.0 seeded sampling; timed decode steps "
                        f"at positions {args.prompt}..{args.prompt + args.steps - 1}",
            "batch": args.batch, "prompt": args.prompt, "context": config.context, "width": config.width,
            "heads": config.heads, "layers": config.layers, "mesh_depth": config.attention_mesh_depth,
            "vocab": config.vocab_size, "temperature": temperature, "init": "reference seed 7",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "persistent_decode_kernel<4, 2, 16, 9, 64> (one launch = all timed steps)",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_calibration": None if not pmc else {
                "fetch_factor": round(pmc["FETCH_SIZE_factor"], 4), "write_factor": round(pmc["WRITE_SIZE_factor"], 4),
                "fetch_bytes": round(pmc["FETCH_SIZE"]), "write_bytes": round(pmc["WRITE_SIZE"])},
            "algorithmic_bytes_per_launch": round(total_bytes),
            "algorithmic_bytes_per_step": round(total_bytes / args.steps),
            "avg_launch_us": round(ms * 1000.0, 1),
        },
        "wall_ms_timed_region": round(wall_ms, 3),
    }
    result["batch1"] = batch1_figure(hip)
    # Measured copy roofline of this box (read + write bytes of a plain copy kernel).
    result["copy_gbps"] = round(G.copy_bandwidth(1 << 30, 10), 1)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(config, prompts, args.steps, temperature, args.cpu_budget)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
