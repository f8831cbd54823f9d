"""Decode throughput of the MI355X Mesh GPT generate path.

Workload ("mid"): vocabulary 256, width 512, 8 heads x 64,
6 blocks, butterfly meshes of depth 9, context 1024, batch 32, 64-token
uniform-random prompts (Random::new(7).index(256)), temperature 1.0 with
per-sequence seeds 7+b; seeded reference initialisation (seed 7).

A bench step is one whole config-3 decode: 512 decode steps of all 32
sequences (positions 64..575, 16384 tokens), in one launch of the persistent
decode kernel.  The prompts are prefilled once, untimed; before each step the
decode state is rewound to the prefill's (lengths and sampler states, two tiny
device copies: mg_decode_rewind), so every step decodes the same 16384 tokens
from inputs resident in HBM.  `value` is tokens/s over the K timed steps by
the host clock between device synchronisations; the roofline divides the
algorithmic HBM bytes of one launch by the launch's average duration from HIP
events that the library records on the model's stream right before and after
the kernel (mg_last_call_ms); avg_call_us adds the launch and the host's
return from the call's synchronisation.

Beside the headline: the first 20 decode steps alone (the latency-bound
short-context end), config 1 at batch 1, config 2's single 9409-row prefill,
config 4's 8192-token prefill and long-context decode, config 5's batch-256
decode, the training step on the reference's training benchmark
(mesh-gpt-bench defaults, ms per AdamW update against its published 5.759 ms),
config 3 with BASELINE.json's N(0, 0.5) weights, the measured copy bandwidth of
the box, HBM traffic from rocprofv3 counters, and the CPU baselines: the
KV-cached f32 decode on the host's threads (config 3's whole workload, a
config-5 sample), the f64 oracle's KV-cached decode on one core, and the
reference's full-window semantics on one core (config 1).
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

HBM_PEAK_GBPS = 8000.0      # MI355X HBM3E, published
FP32_PEAK_TFLOPS = 157.3    # MI355X FP32 (vector with packed FP32, and matrix), published
METRIC = "decode tokens/sec @1 GPU (batch 1 and 32) + % of HBM roofline per decode step"
KERNEL = "persistent_decode_kernel"
DECODE_STEPS = 512          # config 3: decode steps per sequence
PROBE_COPY_BYTES = 256 << 20


class Hip:
    """hipEvent timing on a given stream through libamdhip64."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
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


def step_bytes(config, batch, position):
    """Algorithmic HBM bytes of one decode step of every sequence at `position`
    (all layers): the `position` cached K and V rows read (the current row's
    key and value stay on chip), the new rows appended, the mesh weights, the
    tied head table and the token ids."""
    w, layers = config.width, config.layers
    meshes = 4 * config.attention_mesh_depth + config.ffn_mesh_depth
    return (batch * layers * 2 * w * 4 * position + batch * layers * 2 * w * 4
            + 8 * w * layers * meshes + 4 * config.vocab_size * w + 4 * batch)


def decode_bytes(config, batch, first, steps):
    return float(sum(step_bytes(config, batch, p) for p in range(first, first + steps)))


def timed_decode(hip, model, steps):
    """model.decode(steps) bracketed by HIP events on the model's stream (ms):
    the call's device work, its launch and the host's return from its
    synchronisation."""
    stream = model.stream()
    start, stop = hip.event(), hip.event()
    hip.record(start, stream)
    model.decode(steps)
    hip.record(stop, stream)
    return hip.elapsed_ms(start, stop)


def timed_launch(hip, model, steps):
    """(kernel ms, call ms) of model.decode(steps) in one persistent launch:
    the library's HIP events recorded on the model's stream right before and
    after the kernel (mg_last_call_ms), and timed_decode's bracket of the
    whole call."""
    call = timed_decode(hip, model, steps)
    return model.last_call_ms(), call


def cpu_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def host_threads():
    """The host threads the CPU baselines use: OMP_NUM_THREADS when set (the
    GPU box sets it to its CPU share, 16), else the cores this process may run
    on, at most 16."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, min(16, len(os.sched_getaffinity(0))))


def oracle_config(config):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    return O, O.config(**{k: v for k, v in config.as_dict().items() if k != "long_context"})


def cpu_f32_mode(name, prompts, steps, temperature, threads, sample):
    """cpu-f32-kv: the KV-cached f32 decode of oracle/cpu_f32_decode.c, one
    sequence a thread on `threads` host threads; decode steps only."""
    config = G.named_config(name)
    O, o = oracle_config(config)
    params = O.initialize(o, 7)
    _, seconds = O.cpu_generate_f32(o, params, prompts, steps, temperature, 7, threads)
    tokens = prompts.shape[0] * steps
    return {"mode": "cpu-f32-kv", "workload": name, "value": round(tokens / seconds, 1), "unit": "tokens/s",
            "cores": threads, "cpu": cpu_name(), "sample": sample,
            "us_per_decode_step": round(1e6 * seconds / steps, 1)}


def cpu_baseline(config, prompts, steps, temperature, budget_s):
    """The CPU baselines, timed on this host (bench.py's cpu_baseline leg).
    `value` is cpu-f32-kv on config 3's whole workload (all 32 sequences, all
    512 steps, on host_threads() threads); `modes` adds cpu-f32-kv on a
    config-5 sample, the f64 oracle's KV-cached decode on one core (whole
    config-3 sequences within budget_s), and the reference's own semantics on
    one core (the f64 oracle recomputing the whole window for every token, as
    gpu.rs:2025-2027 and reference.rs:49-59 do) over config 1's whole run."""
    O, o = oracle_config(config)
    params = O.initialize(o, 7)
    threads = host_threads()
    modes = [cpu_f32_mode("mid", prompts, steps, temperature, threads,
                          f"config 3: all {prompts.shape[0]} sequences, {prompts.shape[1]}-token prompts then all "
                          f"{steps} decode steps at T={temperature}; decode time only")]
    high = G.random_prompts(256, 256, 128, 7)[:32]
    modes.append(cpu_f32_mode("high", high, 64, 0.0, threads,
                              "config 5: 32 of its 256 sequences (two per thread), 128-token prompts then 64 "
                              "greedy decode steps (positions 128..191); decode time only"))
    tokens, seconds, done = 0, 0.0, 0
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
    modes.append({"mode": "oracle-f64-kv", "workload": "mid", "value": round(tokens / seconds, 2),
                  "unit": "tokens/s", "cores": 1, "cpu": cpu_name(),
                  "sample": f"config 3: {done} of {prompts.shape[0]} sequences, each its {prompts.shape[1]}-token "
                            f"prompt then {steps} decode steps; decode time only"})
    tiny = G.named_config("tiny")
    Ot, ot = oracle_config(tiny)
    tp = G.random_prompts(64, 1, 16, 7)[0]
    t0 = time.perf_counter()
    Ot.generate(ot, Ot.initialize(ot, 7), tp, 128, 0.0, 7, cached=False)
    seconds1 = time.perf_counter() - t0
    modes.append({"mode": "oracle-f64-window", "workload": "tiny", "value": round(128 / seconds1, 1),
                  "unit": "tokens/s", "cores": 1, "cpu": cpu_name(),
                  "us_per_token": round(1e6 * seconds1 / 128, 1),
                  "sample": "config 1: the whole run, a 16-token prompt then 128 greedy tokens, each from a "
                            "full-window f64 forward (the reference's generate semantics, no KV cache)"})
    first = modes[0]
    return {"value": first["value"], "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"cpu-f32-kv, {first['sample']}; {cpu_name()}", "modes": modes}


def pmc_traffic(args):
    """HBM bytes of one bench-step launch, from two rocprofv3 --pmc runs of a
    child process (FETCH_SIZE, then WRITE_SIZE), each scaled by the same
    counter on a plain copy kernel of known size.  Every run's return code is
    reported; a failed run is not repeated."""
    rocprof = "/opt/rocm/bin/rocprofv3"
    report = {"runs": []}
    if not os.path.exists(rocprof):
        report["error"] = "rocprofv3 not found"
        return report
    import csv

    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="mg_pmc_")
        cmd = ["timeout", "-s", "KILL", "90", rocprof, "--pmc", counter, "-d", out, "-o", "pmc",
               "--output-format", "csv", "--", sys.executable, os.path.abspath(__file__), "--probe"]
        res = subprocess.run(cmd, cwd="/tmp", capture_output=True, text=True)
        hits, copy = [], []
        for path in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for row in csv.DictReader(f):
                    name = row.get("Kernel_Name", "")
                    value = float(row.get("Counter_Value", "nan"))
                    if KERNEL in name and "<4, 2, 16, 9, 64>" in name:
                        hits.append(value)
                    elif "calibration_copy" in name:
                        copy.append(value)
        # rocprofv3 can end with a segmentation fault after its tool
        # finalisation when the program made cooperative launches; the
        # counter file is complete by then, so the rows decide.
        report["runs"].append({"counter": counter, "rc": res.returncode, "kernel_rows": len(hits),
                               "copy_rows": len(copy)})
        if not hits or not copy:
            report["error"] = f"{counter}: no counter rows (rc {res.returncode}): {res.stderr[-300:]}"
            return report
        factor = (PROBE_COPY_BYTES / 1024.0) / float(np.mean(copy))
        report[counter] = float(np.mean(hits)) * factor * 1024.0
        report[counter + "_factor"] = factor
    return report


def probe():
    """Child process under rocprofv3 --pmc: one bench step (the prefill, then
    the 512-step decode launch) and one plain copy of known size."""
    config = G.named_config("mid")
    prompts = G.random_prompts(256, 32, 64, 7)
    with G.MeshGpt(0, config, 7, max_batch=32) as model:
        model.prefill(prompts, 1.0, 7, reserve=64 + 1 + DECODE_STEPS)
        model.decode(DECODE_STEPS)
    G.calibration_copy(PROBE_COPY_BYTES)


def batch1_figure(hip, steps=128):
    """batch 1, 16-token prompt, greedy decode 128 tokens."""
    config = G.named_config("tiny")
    prompts = G.random_prompts(64, 1, 16, 7)
    with G.MeshGpt(0, config, 7) as model:
        model.prefill(prompts, 0.0, 7, reserve=16 + 1 + steps)
        model.decode(steps)  # warm-up
        model.rewind()
        ms = timed_decode(hip, model, steps)
    return {"workload": "config 1 (tiny): V64 W128 H4x32 L2 butterfly depth 7, ctx 256, batch 1, "
                        "16-token prompt, 128 greedy decode steps (one persistent launch)",
            "tokens_per_s": round(steps / (ms / 1000.0), 1), "us_per_token": round(1000.0 * ms / steps, 2)}


def symbolic_figure():
    """one prefill of all 9409 'a + b =' rows, last-position
    logits over the 99 tokens (the grok evaluation's forward)."""
    config = G.named_config("symbolic")
    a, b = np.meshgrid(np.arange(97), np.arange(97), indexing="ij")
    x = np.stack([a.ravel(), np.full(a.size, 97), b.ravel(), np.full(a.size, 98)], axis=1).astype(np.uint32)
    with G.MeshGpt(0, config, 7) as model:
        model.logits(x.ravel(), 4, last_only=True)  # warm-up (workspace growth)
        times = []
        for _ in range(5):
            model.logits(x.ravel(), 4, last_only=True)
            times.append(model.last_call_ms())
    ms = float(np.median(times))
    rows, W, L = x.size, config.width, config.layers
    meshes = 4 * rows * W * L * (4 * config.attention_mesh_depth + config.ffn_mesh_depth)
    hd = W // config.heads
    attention = 9409 * L * config.heads * 2 * hd * 4 * 5
    head = 2 * 9409 * W * config.vocab_size
    flops = meshes + attention + head
    return {"workload": "config 2 (symbolic): V99 W128 H4x32 L2 neighbor A4 F6, 9409 rows of 4 tokens, "
                        "last-position logits; kernel time (HIP events, host copies excluded), median of 5",
            "us": round(1000.0 * ms, 1), "flop": flops,
            "tflops": round(flops / (ms / 1000.0) / 1e12, 3),
            "fp32_frac": round(flops / (ms / 1000.0) / 1e12 / FP32_PEAK_TFLOPS, 4)}


def long_figure(hip, decode_steps=256):
    """batch 8, 8192-token prefill, then 256 greedy decode
    steps over 8192..8447 keys."""
    config = G.named_config("long")
    prompts = G.random_prompts(256, 8, 8192, 7)
    with G.MeshGpt(0, config, 7, max_batch=8) as model:
        model.prefill(prompts, 0.0, 7, reserve=8192 + 1 + decode_steps)
        prefill_ms = model.last_call_ms()
        model.decode(decode_steps)  # warm-up
        model.rewind()
        ms = timed_decode(hip, model, decode_steps)
    W, L, H = config.width, config.layers, config.heads
    hd, n = W // H, 8192
    attention = 8 * L * H * 2 * hd * n * (n + 1)
    meshes = 4 * 8 * n * W * L * (4 * config.attention_mesh_depth + config.ffn_mesh_depth)
    nbytes = decode_bytes(config, 8, 8192, decode_steps)
    return {"workload": "config 4 (long): V256 W512 H8x64 L4 butterfly depth 9, ctx 8448, batch 8, "
                        "8192-token prompts, 256 greedy decode steps",
            "prefill_ms": round(prefill_ms, 3),
            "prefill_tflops": round((attention + meshes) / (prefill_ms / 1000.0) / 1e12, 2),
            "prefill_attention_flop": attention, "prefill_mesh_flop": meshes,
            "decode_tokens_per_s": round(8 * decode_steps / (ms / 1000.0), 1),
            "decode_us_per_step": round(1000.0 * ms / decode_steps, 2),
            "decode_hbm_frac": round(nbytes / (ms / 1000.0) / 1e9 / HBM_PEAK_GBPS, 4)}


def high_figure(hip, decode_steps=1024):
    """batch 256, W1024 L12, 128-token prompts, all 1024
    greedy decode steps (positions 128..1151)."""
    config = G.named_config("high")
    prompts = G.random_prompts(256, 256, 128, 7)
    with G.MeshGpt(0, config, 7, max_batch=256) as model:
        model.prefill(prompts, 0.0, 7, reserve=128 + 1 + decode_steps)
        prefill_ms = model.last_call_ms()
        model.decode(decode_steps)  # warm-up and graph capture
        model.rewind()
        ms = timed_decode(hip, model, decode_steps)
    nbytes = decode_bytes(config, 256, 128, decode_steps)
    return {"workload": "config 5 (high): V256 W1024 H16x64 L12 butterfly depth 10, ctx 2048, batch 256, "
                        f"128-token prompts, greedy decode steps at positions 128..{127 + decode_steps}",
            "prefill_ms": round(prefill_ms, 3),
            "decode_tokens_per_s": round(256 * decode_steps / (ms / 1000.0), 1),
            "decode_us_per_step": round(1000.0 * ms / decode_steps, 2),
            "decode_hbm_frac": round(nbytes / (ms / 1000.0) / 1e9 / HBM_PEAK_GBPS, 4)}


def normal_figure(hip, timed=2):
    """Config 3 as the headline (batch 32, 64-token prompts, 512 decode steps
    at T=1) with BASELINE.json's N(0, 0.5) weights (mg_normal_parameters, seed
    7) instead of the reference's seeded initialisation."""
    config = G.named_config("mid")
    prompts = G.random_prompts(config.vocab_size, 32, 64, 7)
    with G.MeshGpt(0, config, 7, max_batch=32) as model:
        model.set_parameters(G.normal_parameters(config, 7, 0.5))
        model.prefill(prompts, 1.0, 7, reserve=64 + 1 + DECODE_STEPS)
        model.decode(DECODE_STEPS)  # warm-up
        ms = []
        for _ in range(timed):
            model.rewind()
            ms.append(timed_decode(hip, model, DECODE_STEPS))
    avg = float(np.mean(ms))
    nbytes = decode_bytes(config, 32, 64, DECODE_STEPS)
    return {"workload": "config 3 with N(0, 0.5) weights (sigma 0.5, the reference's Box-Muller draw on "
                        "Random::new(7)): batch 32, 64-token prompts, 512 decode steps at T=1",
            "tokens_per_s": round(32 * DECODE_STEPS / (avg / 1000.0), 1),
            "us_per_decode_step": round(1000.0 * avg / DECODE_STEPS, 2),
            "hbm_frac": round(nbytes / (avg / 1000.0) / 1e9 / HBM_PEAK_GBPS, 4)}


def training_figure(steps=30, warmup=10, trials=3):
    """The reference's training benchmark (src/bin/mesh-gpt-bench.rs:29-237,
    timing protocol docs/cuda-performance.md:25-35): add mod 97 with the seeded
    half split, the first 512 training equations (i % split), W128 H4 L2 A4 F6
    V99, context 4, AdamW lr 0.001, weight decay 1, betas 0.9/0.98; each trial
    restores the initial weights, runs `warmup` untimed updates, then times
    `steps` updates by the host clock, including the final parameter download."""
    config = G.GptConfig(vocab_size=99, context=4, width=128, heads=4, layers=2)
    n_train, _ = G.equation_split()
    inputs, targets = G.equation_batch(np.arange(512) % n_train)
    opts = G.AdamW(learning_rate=0.001, weight_decay=1.0, beta2=0.98)
    results = []
    with G.MeshGpt(0, config, 7) as model:
        initial = model.parameters()
        for _ in range(trials):
            model.set_parameters(initial)
            for _ in range(warmup):
                model.train_batch(inputs, targets, 4, opts)
            model.parameters()
            t0 = time.perf_counter()
            first = last = 0.0
            for step in range(steps):
                last = model.train_batch(inputs, targets, 4, opts)
                if step == 0:
                    first = last
            model.parameters()
            ms = 1000.0 * (time.perf_counter() - t0) / steps
            results.append((ms, first, last))
    ms = float(np.median([r[0] for r in results]))
    return {"workload": "reference training benchmark (mesh-gpt-bench defaults): add mod 97, 512 training equations, "
                        "W128 H4 L2 A4 F6 V99 ctx 4, AdamW lr 1e-3 wd 1 betas 0.9/0.98; "
                        f"{trials} trials of {warmup} warm-up + {steps} timed updates, parameter download included",
            "ms_per_update": round(ms, 4), "trials_ms": [round(r[0], 4) for r in results],
            "tokens_per_s": round(len(inputs) * 1000.0 / ms, 1),
            "ce_first_last": [round(results[0][1], 6), round(results[0][2], 6)],
            "published_ms_per_update": 5.759,
            "published_hardware": "RTX 3050 Laptop GPU (docs/cuda-performance.md:36-61)",
            "speedup_vs_published": round(5.759 / ms, 2)}


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=5, help="timed whole 512-step decodes")
    parser.add_argument("--warmup", type=int, default=2)
    parser.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-pmc", action="store_true")
    parser.add_argument("--no-extra", action="store_true", help="config 3 only")
    parser.add_argument("--only", choices=["batch1", "config2", "config4", "config5", "normal", "training",
                                           "cpu"],
                        help="print only that figure (for profiling one workload)")
    parser.add_argument("--calibrate", action="store_true",
                        help="with --only: a plain copy of 256 MiB after the figure (the scale of counter runs)")
    parser.add_argument("--probe", action="store_true", help=argparse.SUPPRESS)
    args = parser.parse_args()

    if args.probe:
        probe()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "decode would shard by sequence with no per-step exchange between GPUs.", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1:
        sys.exit("--steps must be at least 1")

    if args.only:
        mid = G.named_config("mid")
        figures = {"batch1": lambda: batch1_figure(Hip()), "config2": symbolic_figure,
                   "config4": lambda: long_figure(Hip()), "config5": lambda: high_figure(Hip()),
                   "normal": lambda: normal_figure(Hip()), "training": training_figure,
                   "cpu": lambda: cpu_baseline(mid, G.random_prompts(256, 32, 64, 7), DECODE_STEPS, 1.0,
                                               args.cpu_budget)}
        print(json.dumps({args.only: figures[args.only]()}))
        if args.calibrate:
            G.calibration_copy(PROBE_COPY_BYTES)
        return
    # The counter runs go first, while this process has not touched the GPU:
    # the profiled child is then the only process on it.
    pmc = None if args.no_pmc else pmc_traffic(args)

    config = G.named_config("mid")
    batch, prompt_len, temperature = 32, 64, 1.0
    prompts = G.random_prompts(config.vocab_size, batch, prompt_len, 7)
    hip = Hip()
    with G.MeshGpt(0, config, 7, max_batch=batch) as model:
        model.prefill(prompts, temperature, 7, reserve=prompt_len + 1 + DECODE_STEPS)
        for _ in range(args.warmup):
            model.rewind()
            model.decode(DECODE_STEPS)
        hip.synchronize()
        launch_ms, call_ms = [], []
        t0 = time.perf_counter()
        for _ in range(args.steps):
            model.rewind()
            kernel, call = timed_launch(hip, model, DECODE_STEPS)
            launch_ms.append(kernel)
            call_ms.append(call)
        hip.synchronize()
        wall_s = time.perf_counter() - t0
        # The latency-bound end alone: the first 20 decode steps (median of 5 launches).
        early = []
        for _ in range(5):
            model.rewind()
            early.append(timed_launch(hip, model, 20))
        early_ms = float(np.median([e[0] for e in early]))
        early_call_ms = float(np.median([e[1] for e in early]))

    avg_ms = float(np.mean(launch_ms))
    launch_bytes = decode_bytes(config, batch, prompt_len, DECODE_STEPS)
    gbps = launch_bytes / (avg_ms / 1000.0) / 1e9
    early_bytes = decode_bytes(config, batch, prompt_len, 20)
    tokens = batch * DECODE_STEPS * args.steps

    result = {
        "metric": METRIC,
        "value": round(tokens / wall_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * wall_s / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "config 3 (mid): V256 W512 H8x64 L6 butterfly depth 9, ctx 1024, batch 32, "
                        "64-token uniform-random prompts, T=1.0 seeded sampling; one step = all 512 decode "
                        "steps of the batch (positions 64..575, 16384 tokens) from the rewound prefill state",
            "batch": batch, "prompt": prompt_len, "decode_steps_per_step": DECODE_STEPS,
            "context": config.context, "width": config.width, "heads": config.heads, "layers": config.layers,
            "mesh_depth": config.attention_mesh_depth, "vocab": config.vocab_size, "temperature": temperature,
            "init": "reference seed 7",
        },
        "us_per_decode_step": round(1000.0 * avg_ms / DECODE_STEPS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "persistent_decode_kernel<4, 2, 16, 9, 64> (one launch = one bench step)",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": round(launch_bytes),
            "avg_launch_us": round(avg_ms * 1000.0, 1),
            "launch_us": [round(m * 1000.0, 1) for m in launch_ms],
            "timing": "HIP events recorded by the library on the model's stream right before and after "
                      "the kernel launch (mg_last_call_ms)",
            "avg_call_us": round(float(np.mean(call_ms)) * 1000.0, 1),
        },
        "early_slice": {
            "positions": f"{prompt_len}..{prompt_len + 19}",
            "us_per_decode_step": round(1000.0 * early_ms / 20, 2),
            "tokens_per_s": round(batch * 20 / (early_ms / 1000.0), 1),
            "hbm_frac": round(early_bytes / (early_ms / 1000.0) / 1e9 / HBM_PEAK_GBPS, 4),
            "timing": "kernel events, median of 5 launches of 20 steps",
            "call_us_per_decode_step": round(1000.0 * early_call_ms / 20, 2),
        },
    }
    if pmc is not None:
        result["roofline"]["traffic_calibration"] = pmc
        if "FETCH_SIZE" in pmc and "WRITE_SIZE" in pmc:
            result["roofline"]["traffic"] = round(pmc["FETCH_SIZE"] + pmc["WRITE_SIZE"])
    result["batch1"] = batch1_figure(hip)
    if not args.no_extra:
        result["config2"] = symbolic_figure()
        result["config4"] = long_figure(hip)
        result["config5"] = high_figure(hip)
        result["config3_normal_init"] = normal_figure(hip)
        result["training"] = training_figure()
    # Measured copy roofline of this box (read + write bytes of a plain copy kernel).
    result["copy_gbps"] = round(G.copy_bandwidth(1 << 30, 10), 1)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(config, prompts, DECODE_STEPS, temperature, args.cpu_budget)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
