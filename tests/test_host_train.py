"""Host-side pieces of the training path (no GPU): the equation dataset the
training benchmark and the grok evaluation feed (src/gpt/grokking.rs:116-258),
the text dataset of `mesh-gpt train` (src/gpt/text.rs:58-108), the AdamW
defaults (src/gpt/config.rs:258-276) and the `mesh-gpt train` rejections that
come before any device work (src/bin/mesh-gpt.rs:173-184, geometry.rs:24-55).

The datasets are checked against the oracle's restatements, which the
published step-0 cross-entropies pin (tests/test_oracle.py), for every
operation; the split sizes are the published 4704 / 4705
(docs/grokking.md:14-15).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import grokking_abmod_amd as G
import oracle_lib as O


def oracle_equations(modulus, operation, fraction, seed):
    perm = np.zeros(modulus, np.uint32)
    tr = np.zeros(3 * modulus * modulus, np.uint32)
    va = np.zeros_like(tr)
    nt, nv = ctypes.c_size_t(), ctypes.c_size_t()
    rc = O.lib().og_equations(modulus, operation, fraction, seed, O.ptr(perm, O._u32p), O.ptr(tr, O._u32p),
                              O.ptr(va, O._u32p), ctypes.byref(nt), ctypes.byref(nv))
    assert rc == 0
    return perm, tr[:3 * nt.value].reshape(-1, 3), va[:3 * nv.value].reshape(-1, 3)


def test_published_split_sizes():
    assert G.equation_split() == (4704, 4705)


@pytest.mark.parametrize("operation", range(10))
def test_batches_equal_the_oracle(operation):
    modulus, fraction, seed = 31, 0.4, 11
    perm, train, valid = oracle_equations(modulus, operation, fraction, seed)
    assert G.equation_split(modulus, operation, fraction, seed) == (len(train), len(valid))
    for validation, split in ((False, train), (True, valid)):
        idx = np.arange(len(split))[::-1]
        x, y = G.equation_batch(idx, validation, modulus, operation, fraction, seed)
        rows = split[idx]
        want_x = np.stack([perm[rows[:, 0]], np.full(len(idx), modulus), perm[rows[:, 1]],
                           np.full(len(idx), modulus + 1)], 1).reshape(-1)
        ign = np.full(len(idx), G.IGNORE_TARGET, np.uint32)
        want_y = np.stack([ign, ign, ign, perm[rows[:, 2]]], 1).reshape(-1)
        assert np.array_equal(x, want_x) and np.array_equal(y, want_y)


def test_dataset_rejections_carry_the_reference_messages():
    cases = [
        (lambda: G.equation_split(96), "modulus must be a prime in 2..254 (two vocabulary slots are reserved)"),
        (lambda: G.equation_split(97, 0, 0.0), "train fraction must be finite and strictly between 0 and 1"),
        (lambda: G.equation_split(97, 0, 1.0), "train fraction must be finite and strictly between 0 and 1"),
        (lambda: G.equation_split(257), "modulus must be a prime in 2..254 (two vocabulary slots are reserved)"),
        (lambda: G.equation_split(2, 0, 0.1), "split needs at least two training equations and one validation equation"),
        (lambda: G.equation_batch([4704]), "equation index is outside the split"),
        (lambda: G.equation_batch([]), "equation batches need 1..32768 examples"),
    ]
    for call, message in cases:
        with pytest.raises(G.MeshGptError) as err:
            call()
        assert message in str(err.value)


def test_adamw_defaults():
    a = G.AdamW()
    assert (a.learning_rate, a.weight_decay, a.beta1, a.beta2, a.epsilon) == tuple(
        float(np.float32(v)) for v in (0.003, 0.01, 0.9, 0.999, 1e-8))


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CORPUS = os.path.join(ROOT, "tests", "golden", "mesh-gpt-demo.txt")


def demo_tokens():
    with open(CORPUS, encoding="utf-8") as f:
        text = f.read()
    chars = sorted(set(text))
    index = {ch: i for i, ch in enumerate(chars)}
    return np.array([index[ch] for ch in text], dtype=np.uint32), len(chars)


@pytest.mark.parametrize("validation", [False, True])
@pytest.mark.parametrize("sequence,batch,seed", [(32, 8, 7), (32, 8, 101), (5, 3, 2 ** 64 - 1), (1, 40, 12345)])
def test_text_batches_equal_the_oracle(validation, sequence, batch, seed):
    tokens, V = demo_tokens()
    cfg = G.GptConfig(vocab_size=V, context=32)
    x, y = G.text_batch(tokens, cfg, validation, sequence, batch, seed)
    want_x, want_y = O.text_batch(tokens, validation, sequence, batch, seed)
    assert np.array_equal(x, want_x) and np.array_equal(y, want_y)
    # Windows stay inside their split and targets are the next tokens.
    split = tokens.size * 9 // 10
    corpus = tokens[split:] if validation else tokens[:split]
    for b in range(batch):
        row = x[b * sequence:(b + 1) * sequence]
        starts = [i for i in range(corpus.size - sequence) if np.array_equal(corpus[i:i + sequence], row)]
        assert any(np.array_equal(corpus[i + 1:i + sequence + 1], y[b * sequence:(b + 1) * sequence])
                   for i in starts)


def test_text_dataset_rejections_carry_the_reference_messages():
    tokens, V = demo_tokens()
    cfg = G.GptConfig(vocab_size=V, context=32)
    cases = [
        (lambda: G.text_batch(tokens, G.GptConfig(vocab_size=V - 1, context=32), False, 32, 8, 7),
         "dataset has invalid token IDs"),
        (lambda: G.text_batch(tokens[:300], cfg, False, 32, 8, 7),
         "corpus is too short for a 90/10 split at this context length"),
        (lambda: G.text_batch(tokens, cfg, False, 0, 8, 7), "invalid dataset batch dimensions"),
        (lambda: G.text_batch(tokens, cfg, False, 32, 0, 7), "invalid dataset batch dimensions"),
        (lambda: G.text_batch(tokens, cfg, False, 32, 4097, 7), "invalid dataset batch dimensions"),
        (lambda: G.text_batch(tokens, cfg, True, tokens.size - tokens.size * 9 // 10, 1, 7),
         "invalid dataset batch dimensions"),
        (lambda: G.text_batch(tokens, G.GptConfig(vocab_size=V, context=32, heads=3), False, 32, 8, 7),
         "heads must be in 1..64 and divide width"),
    ]
    for call, message in cases:
        with pytest.raises(G.MeshGptError) as err:
            call()
        assert message in str(err.value)


def cli(*args):
    return subprocess.run([G.CLI_PATH, *args], capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("args,message", [
    (["--steps", "0"], "steps and report_every must be positive"),
    (["--report-every", "0"], "steps and report_every must be positive"),
    (["--learning-rate", "0"], "learning_rate must be positive and weight_decay nonnegative; both must be finite"),
    (["--weight-decay", "-1"], "learning_rate must be positive and weight_decay nonnegative; both must be finite"),
    (["--learning-rate", "inf"], "learning_rate must be positive and weight_decay nonnegative; both must be finite"),
    (["--prompt", ""], "generation prompt must not be empty"),
    (["--temperature", "-1"], "temperature must be finite and nonnegative"),
    (["--heads", "3"], "heads must be in 1..64 and divide width"),
    (["--context", "5000"], "context must be in 1..4096"),
    (["--rope", "2"], "--rope requires 0 or 1"),
    (["--qk-norm", "x"], "invalid value for --qk-norm: x"),
    (["--embedding-form", "cube"], "invalid value for --embedding-form: cube"),
    (["--embedding-order", "x"], "invalid value for --embedding-order: x"),
    (["--embedding-norm", "l2"], "invalid value for --embedding-norm: l2"),
    (["--embedding-norm"], "missing value for --embedding-norm"),
    (["--unknown"], "unknown option: --unknown; use --help"),
    (["--batch", "5000"], "invalid dataset batch dimensions"),
    (["--batch", "0"], "invalid dataset batch dimensions"),
])
def test_cli_train_rejections(args, message):
    """Each is raised before any device work, so no GPU is needed."""
    res = cli("train", "--dataset", CORPUS, *args)
    assert res.returncode == 1 and res.stdout == ""
    assert res.stderr == f'Error: "{message}"\n'


def test_cli_help_lists_the_training_and_geometry_flags():
    res = cli("--help")
    assert res.returncode == 0
    for flag in ("--steps", "--learning-rate", "--weight-decay", "--report-every", "--embedding-form",
                 "--embedding-order", "--embedding-frequency", "--embedding-harmonics", "--equiangular-overlap",
                 "--embedding-norm", "--freeze-embedding", "--preserve-features", "--geometry-seed", "--rope",
                 "--qk-norm", "--xsa"):
        assert flag in res.stdout, flag


BENCH_PATH = os.path.join(os.path.dirname(G.CLI_PATH), "mesh-gpt-bench")


@pytest.mark.parametrize("args,message", [
    (["--steps", "0"], "steps/trials/batch must be positive, with at most 131072 token rows"),
    (["--trials", "0"], "steps/trials/batch must be positive, with at most 131072 token rows"),
    (["--batch", "40000"], "steps/trials/batch must be positive, with at most 131072 token rows"),
    (["--heads", "16", "--width", "128"], "benchmark requires width <=1024 and <=8 heads"),
    (["--width", "2048", "--heads", "8"], "benchmark requires width <=1024 and <=8 heads"),
    (["--context", "256", "--width", "256"], "benchmark context must be <=128, or <=4096 with width <=128"),
    (["--heads", "3"], "heads must be in 1..64 and divide width"),
    (["--steps", "x"], "invalid value for --steps: x"),
    (["--bogus"], "unknown benchmark option: --bogus"),
])
def test_bench_binary_rejections(args, message):
    """mesh-gpt-bench (src/bin/mesh-gpt-bench.rs:29-103) refuses these before any device work."""
    res = subprocess.run([BENCH_PATH, *args], capture_output=True, text=True, timeout=60)
    assert res.returncode == 1 and res.stdout == ""
    assert res.stderr == f'Error: "{message}"\n'


def test_bench_binary_help():
    res = subprocess.run([BENCH_PATH, "--help"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0
    for flag in ("--steps", "--warmup", "--trials", "--batch", "--width", "--heads", "--context", "--layers",
                 "--attention-depth", "--ffn-depth", "--device", "--output"):
        assert flag in res.stdout


@pytest.mark.parametrize("args,message", [
    (["--steps", "5", "--epochs", "1"], "choose either --epochs or --steps"),
    (["--operation", "pow"], "invalid value for --operation: pow"),
    (["--modulus", "96"], "modulus must be a prime in 2..254 (two vocabulary slots are reserved)"),
    (["--train-fraction", "1"], "train fraction must be finite and strictly between 0 and 1"),
    (["--report-every", "0"], "steps, report interval, and evaluation batch must be positive"),
    (["--eval-batch", "0"], "steps, report interval, and evaluation batch must be positive"),
    (["--init-gain", "0"], "initialization gains must be finite and positive"),
    (["--embedding-output-gain", "nan"], "initialization gains must be finite and positive"),
    (["--workspace-cache", "4"], "workspace capacity must be in 1..3"),
    (["--stop-validation-accuracy", "1.5"], "validation stop accuracy must be in (0, 1]"),
    (["--qk-signs", "2"], "Q/K sign initialization must be 0 or 1"),
    (["--learning-rate", "0"],
     "AdamW requires finite positive learning rate/epsilon, nonnegative decay, and betas in [0, 1)"),
    (["--embedding-init-unit"],
     "initial unit normalization requires table embeddings, embedding-norm none, and no protected features"),
    (["--batch", "5000"], "invalid equation minibatch size"),
    (["--width", "2048"], "grokking requires width <=1024"),
    (["--embedding-form", "cube"], "invalid value for --embedding-form: cube"),
    (["--bogus"], "unknown grok option: --bogus; use grok --help"),
])
def test_cli_grok_rejections(args, message):
    """`mesh-gpt grok` (src/bin/mesh-gpt/grokking.rs:44-218) refuses these before any device work."""
    res = cli("grok", *args)
    assert res.returncode == 1 and res.stdout == ""
    assert res.stderr == f'Error: "{message}"\n'


def test_cli_grok_help():
    res = cli("grok", "--help")
    assert res.returncode == 0
    for flag in ("--operation", "--modulus", "--train-fraction", "--epochs", "--stop-validation-accuracy",
                 "--eval-batch", "--workspace-cache", "--init-gain", "--embedding-output-gain",
                 "--embedding-init-unit", "--qk-signs", "--embedding-form", "--xsa"):
        assert flag in res.stdout, flag
