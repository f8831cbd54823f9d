"""GPU: the benchmark configurations at their real shapes and lengths.

Each test drives the product through the C ABI and checks it three ways:
against the f64 oracle where the oracle finishes in seconds (token
trajectories under the rounding rule of trajectory.py, logits within
TOL*(1+|ref|)), against a device re-prefill of the device's own tokens
(decode with the KV cache equals recomputing the window: mesh-gpt.rs:387-394's
prefix invariance, used at full size), and persistent decode against the
per-phase kernels.  Prompts are Random::new(7).index(V) draws
(grokking_abmod_amd.random_prompts), as the benchmark's.

Coverage by position: config 3 runs all 512 decode steps (keys 65..576), so
the persistent attention's LDS-ring refills and two-round register tail run;
the W1024/H16 shape runs past 300 keys through the three-slot ring; config 4
prefills 8192 tokens and decodes 256 steps past them.
"""
import json
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import grokking_abmod_amd as G
import oracle_lib as O
from conftest import ROOT, TOL, assert_close
from trajectory import check_trajectory

pytestmark = pytest.mark.gpu


def oracle_config(config):
    return O.config(**{k: v for k, v in config.as_dict().items() if k != "long_context"})


def parallel(fn, items, workers=8):
    # The oracle's ctypes calls release the GIL, so threads run them in parallel.
    with ThreadPoolExecutor(workers) as ex:
        return list(ex.map(fn, items))


def last_row_logits(model):
    return lambda window: model.logits(window, len(window), last_only=True)[0]


def reprefill_last(model, tokens):
    """Device logits of each sequence's last row, recomputed from scratch."""
    batch, n = tokens.shape
    return model.logits(np.ascontiguousarray(tokens).reshape(-1), n, last_only=True)


def assert_same_tokens_or_near_tie(model, got, other, what, gap_tol=1e-5):
    """Two device greedy trajectories agree until a step whose top-2 logit gap
    (device re-prefill) is within gap_tol*(1+|top|); returns tokens compared."""
    compared = 0
    for b in range(got.shape[0]):
        diff = np.nonzero(got[b] != other[b])[0]
        if diff.size == 0:
            compared += got.shape[1]
            continue
        k = int(diff[0])
        row = model.logits(got[b, :k], k, last_only=True)[0].astype(np.float64)
        top = np.sort(row)[-2:]
        assert top[1] - top[0] <= gap_tol * (1 + abs(top[1])), \
            f"{what}: sequence {b} differs at {k} with top-2 gap {top[1] - top[0]:.3g}"
        compared += k
    return compared


def test_config3_full_decode_greedy_matches_oracle():
    # Config 3 shape, greedy: all 512 decode steps (positions 64..575) in one
    # persistent launch; 8 sequences' trajectories against the oracle, 4
    # sequences' last-step logits against the oracle on the device's tokens,
    # and every sequence's last-step logits against a device re-prefill.
    config = G.named_config("mid")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 32, 64, 7)
    expected = parallel(lambda b: O.generate(o, params, prompts[b], 512, 0.0, 7 + b, cached=True), range(8))
    with G.MeshGpt(0, config, 7, max_batch=32) as model:
        got = model.generate_tokens(prompts, 512, 0.0, 7)
        last = model.last_logits(32)
        refs = parallel(lambda b: O.logits(o, params, got[b, :-1], 575)[-1], range(4))
        for b in range(4):
            assert_close(last[b], refs[b], what=f"config-3 step-512 logits, sequence {b}")
        assert_close(last, reprefill_last(model, got[:, :-1]), what="config-3 decode vs re-prefill")
        for b in range(8):
            check_trajectory(o, params, prompts[b], got[b], 0.0, 7 + b, last_row_logits(model),
                             expected=expected[b])


def test_config3_full_decode_sampled_matches_oracle(monkeypatch):
    # Config 3 as benchmarked: T=1.0, seeds 7+b, 512 steps.  The persistent
    # launch and the per-phase kernels each match the oracle (6 sequences),
    # and each one's last-step logits equal a device re-prefill.  (The two
    # paths sum attention in different orders, so a sampled token may differ
    # between them where a draw lies within rounding of a CDF boundary; each
    # is held to the oracle instead.)
    config = G.named_config("mid")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 32, 64, 7)
    expected = parallel(lambda b: O.generate(o, params, prompts[b], 512, 1.0, 7 + b, cached=True), range(6))
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_PERSISTENT", disable)
        with G.MeshGpt(0, config, 7, max_batch=32) as model:
            got = model.generate_tokens(prompts, 512, 1.0, 7)
            assert_close(model.last_logits(32), reprefill_last(model, got[:, :-1]),
                         what=f"config-3 T=1 decode vs re-prefill (per-phase={disable})")
            for b in range(6):
                check_trajectory(o, params, prompts[b], got[b], 1.0, 7 + b, last_row_logits(model),
                                 expected=expected[b])


def test_config3_agent_scope_handoffs_match_xcd_local(monkeypatch):
    # The persistent kernel's agent-scope hand-off protocol (the one a
    # sequence falls back to when its workgroups are not all on one XCD),
    # forced for every sequence with MG_PERSIST_AGENT_SCOPE=1, at config 3's
    # full batch over 200 sampled steps (T=1, keys 65..264): tokens and
    # last-step logits bit-equal to the XCD-local words' run (the same
    # arithmetic in the same order), last-step logits of every sequence equal
    # to a device re-prefill and of two against the oracle.
    config = G.named_config("mid")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 32, 64, 7)
    runs = {}
    for agent in ("0", "1"):
        monkeypatch.setenv("MG_PERSIST_AGENT_SCOPE", agent)
        with G.MeshGpt(0, config, 7, max_batch=32) as model:
            got = model.generate_tokens(prompts, 200, 1.0, 7)
            last = model.last_logits(32)
            runs[agent] = (got, last)
            if agent == "1":
                assert_close(last, reprefill_last(model, got[:, :-1]), what="agent-scope decode vs re-prefill")
                refs = parallel(lambda b: O.logits(o, params, got[b, :-1], got.shape[1] - 1)[-1], range(2))
                for b in range(2):
                    assert_close(last[b], refs[b], what=f"agent-scope step-200 logits, sequence {b}")
    assert np.array_equal(runs["0"][0], runs["1"][0])
    assert np.array_equal(runs["0"][1], runs["1"][1])


@pytest.mark.parametrize("name,batch,prompt,steps,temperature,checked", [
    ("tiny", 1, 16, 128, 0.0, 1), ("mid", 32, 64, 512, 0.0, 4), ("mid", 32, 64, 512, 1.0, 4)],
    ids=["config1-greedy", "config3-greedy", "config3-T1"])
def test_normal_weights_decode_matches_oracle(name, batch, prompt, steps, temperature, checked):
    # BASELINE.json's N(0, 0.5) weights (mg_normal_parameters, seed 7, the
    # reference's Box-Muller draw) at configs 1 and 3: trajectories of
    # `checked` sequences against the oracle's decode on the same weights,
    # last-step logits of two against the oracle and of all against a device
    # re-prefill.
    config = G.named_config(name)
    o = oracle_config(config)
    params = O.initialize_normal(o, 7, 0.5)
    prompts = G.random_prompts(config.vocab_size, batch, prompt, 7)
    expected = parallel(lambda b: O.generate(o, params, prompts[b], steps, temperature, 7 + b, cached=True),
                        range(checked))
    with G.MeshGpt(0, config, 7, max_batch=batch) as model:
        weights = G.normal_parameters(config, 7, 0.5)
        assert np.array_equal(weights, params)
        model.set_parameters(weights)
        got = model.generate_tokens(prompts, steps, temperature, 7)
        last = model.last_logits(batch)
        n = got.shape[1] - 1
        refs = parallel(lambda b: O.logits(o, params, got[b, :-1], n)[-1], range(min(2, checked)))
        for b, ref in enumerate(refs):
            assert_close(last[b], ref, what=f"{name} N(0, 0.5) last-step logits, sequence {b}")
        assert_close(last, reprefill_last(model, got[:, :-1]), what=f"{name} N(0, 0.5) decode vs re-prefill")
        for b in range(checked):
            check_trajectory(o, params, prompts[b], got[b], temperature, 7 + b, last_row_logits(model),
                             expected=expected[b])


def test_config3_decode_segments_continue_one_launch():
    # Four persistent launches (150 + 150 + 150 + 61 steps after the prefill's
    # token) produce exactly the tokens of one 511-step launch, and each
    # segment's last-step logits equal a device re-prefill; sequences 0-1
    # against the oracle's logits at every segment end.
    config = G.named_config("mid")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 32, 64, 11)
    with G.MeshGpt(0, config, 7, max_batch=32) as model:
        whole = model.generate_tokens(prompts, 512, 1.0, 3)
        model.prefill(prompts, 1.0, 3, reserve=64 + 512)
        for steps in (150, 150, 150, 61):
            model.decode(steps)
            n = model.sequence_length()
            tokens = model.read_tokens(32, n)
            last = model.last_logits(32)
            assert_close(last, reprefill_last(model, tokens[:, :-1]), what=f"segment ending at {n}")
            refs = parallel(lambda b: O.logits(o, params, tokens[b, :-1], n - 1)[-1], range(2))
            for b in range(2):
                assert_close(last[b], refs[b], what=f"segment ending at {n}, sequence {b}")
        assert np.array_equal(model.read_tokens(32), whole)
        # A rewind repeats the same steps from the prefill's state.
        model.rewind()
        model.decode(511)
        assert np.array_equal(model.read_tokens(32), whole)


def test_width1024_persistent_decode_past_300_keys(monkeypatch):
    # Config 5's row shape (W1024, H16x64, depth 10, butterfly) at batch 4 runs
    # the persistent kernel (forced: at this batch and length the per-phase
    # kernels are the default) with its three-slot ring; 128-token prompts and 200
    # greedy steps reach 327 keys.  Two sequences against the oracle; all four
    # against the per-phase kernels.
    config = G.GptConfig(vocab_size=256, width=1024, heads=16, layers=3, attention_mesh_depth=10,
                         ffn_mesh_depth=10, context=512, connectivity=1)
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 4, 128, 7)
    expected = parallel(lambda b: O.generate(o, params, prompts[b], 200, 0.0, 7 + b, cached=True), range(2))
    runs = {}
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_PERSISTENT", disable)
        monkeypatch.setenv("MG_FORCE_PERSISTENT", "1" if disable == "0" else "0")
        with G.MeshGpt(0, config, 7, max_batch=4) as model:
            got = model.generate_tokens(prompts, 200, 0.0, 7)
            assert_close(model.last_logits(4), reprefill_last(model, got[:, :-1]),
                         what=f"W1024 decode vs re-prefill (per-phase={disable})")
            if disable == "0":
                for b in range(2):
                    check_trajectory(o, params, prompts[b], got[b], 0.0, 7 + b, last_row_logits(model),
                                     expected=expected[b])
                runs["persistent"] = got
            else:
                assert_same_tokens_or_near_tie(model, got, runs["persistent"], "W1024 persistent vs per-phase")


def test_config4_long_context_full_size(monkeypatch):
    # Config 4: batch 8, 8192-token prefill (causal flash attention over
    # 8192 keys), then 256 greedy decode steps to 8448 tokens, the whole
    # extended context.  Last-step logits equal a device re-prefill of all
    # 8448 positions; persistent (forced: the per-phase kernels are the
    # default at this batch and length) and per-phase decode give the same
    # tokens.
    config = G.named_config("long")
    prompts = G.random_prompts(256, 8, 8192, 7)
    runs = {}
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_PERSISTENT", disable)
        monkeypatch.setenv("MG_FORCE_PERSISTENT", "1" if disable == "0" else "0")
        with G.MeshGpt(0, config, 7, max_batch=8) as model:
            got = model.generate_tokens(prompts, 256, 0.0, 7)
            assert got.shape == (8, 8448)
            assert np.array_equal(got[:, :8192], prompts)
            assert_close(model.last_logits(8), reprefill_last(model, got[:, :-1]),
                         what=f"config-4 step-256 logits vs re-prefill (per-phase={disable})")
            if disable == "1":
                assert_same_tokens_or_near_tie(model, got, runs["0"], "config-4 persistent vs per-phase")
            runs[disable] = got


@pytest.mark.parametrize("mfma", ["1", "0"], ids=["mfma", "valu"])
def test_config4_full_prefill_matches_oracle_fixture(mfma, monkeypatch):
    # Config 4's 8192-token prefill against the f64 oracle: the last-row
    # logits of benchmark prompt 0 cut at 1024, 4096 and 8192 tokens
    # (tests/golden/config4_prefill.json, written by make_config4_prefill.py
    # from one oracle forward over all 8192 rows), on the matrix-core flash
    # attention and on the VALU flash kernel.  At 8192 keys the f32 softmax
    # sums differ most from f64; the bound stays TOL * (1 + |ref|).
    with open(os.path.join(ROOT, "tests", "golden", "config4_prefill.json")) as f:
        fixture = json.load(f)
    config = G.named_config("long")
    assert fixture["config"] == config.as_dict()
    prompt = G.random_prompts(256, 8, 8192, 7)[0]
    assert fixture["prompt_sha"] == int(np.bitwise_xor.reduce(
        prompt.astype(np.uint64) * (np.arange(8192, dtype=np.uint64) + 1)))
    monkeypatch.setenv("MG_DISABLE_MFMA_PREFILL", "0" if mfma == "1" else "1")
    with G.MeshGpt(0, config, 7) as model:
        for n, row in fixture["rows"].items():
            got = model.logits(prompt[:int(n)], int(n), last_only=True)[0]
            assert_close(got, np.array(row), what=f"config-4 prefill of {n} tokens, last row")


def test_config4_shape_against_oracle():
    # Config 4's model (W512 L4, context 8448) on a length the oracle covers:
    # one 1024-token prompt and 16 greedy steps.
    config = G.named_config("long")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompt = G.random_prompts(256, 1, 1024, 5)[0]
    expected = O.generate(o, params, prompt, 16, 0.0, 7, cached=True)
    with G.MeshGpt(0, config, 7) as model:
        got = model.generate_tokens(prompt[None, :], 16, 0.0, 7)[0]
        ref = O.logits(o, params, got[:-1], len(got) - 1)[-1]
        assert_close(model.last_logits(1)[0], ref, what="config-4 decode logits")
        check_trajectory(o, params, prompt, got, 0.0, 7, last_row_logits(model), expected=expected)


@pytest.mark.timeout(900)
def test_config5_high_batch_full_size():
    # Config 5 exactly: batch 256, W1024 L12 H16x64, context 2048 (a 48 GiB KV
    # cache), 128-token prompts, all 1024 greedy steps (positions 128..1151)
    # on the per-phase kernels (4864 workgroups exceed co-residency, so no
    # persistent launch), in two slices of 128 sequences on two streams.  The
    # last step's logits of all 256 sequences against a device re-prefill of
    # their 1151 tokens (in chunks within the 131072-row limit), and sequence
    # 0's trajectory and last-step logits against the oracle (its cached
    # decode, and its full forward over the device's tokens).
    config = G.named_config("high")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 256, 128, 7)
    with ThreadPoolExecutor(2) as ex:
        expected = ex.submit(O.generate, o, params, prompts[0], 1024, 0.0, 7, True)
        with G.MeshGpt(0, config, 7, max_batch=256) as model:
            got = model.generate_tokens(prompts, 1024, 0.0, 7)
            assert got.shape == (256, 1152)
            assert np.array_equal(got[:, :128], prompts)
            ref = ex.submit(lambda: O.logits(o, params, got[0, :-1], 1151)[-1])
            last = model.last_logits(256)
            for b0 in range(0, 256, 96):
                assert_close(last[b0:b0 + 96], reprefill_last(model, got[b0:b0 + 96, :-1]),
                             what=f"config-5 step-1024 logits vs re-prefill, sequences {b0}..")
            assert_close(last[0], ref.result(), what="config-5 step-1024 logits, sequence 0")
            check_trajectory(o, params, prompts[0], got[0], 0.0, 7, last_row_logits(model),
                             expected=expected.result())


@pytest.mark.parametrize("temperature,graph", [(0.0, True), (1.0, True), (1.0, False)])
def test_decode_slices_match_one_stream(temperature, graph, monkeypatch):
    # The per-phase decode of a large batch runs as slices of the batch on
    # their own streams (sequences are independent: rows, cache slabs,
    # generator states and tokens are per sequence).  With the attention
    # split count fixed, each sequence's arithmetic is that of one stream, so
    # tokens and final logits must be bit-identical for 1, 2 and 3 slices of
    # the 96 sequences, over three 8-step graph replays or, without graphs,
    # 24 single steps.
    config = G.named_config("mid")
    monkeypatch.setenv("MG_DISABLE_PERSISTENT", "1")
    monkeypatch.setenv("MG_DISABLE_GRAPH", "0" if graph else "1")
    monkeypatch.setenv("MG_DECODE_SPLITS", "2")
    monkeypatch.setenv("MG_ROW_BATCH", "1")
    prompts = G.random_prompts(256, 96, 16, 7)
    results = {}
    for slices in ("1", "2", "3"):
        monkeypatch.setenv("MG_DECODE_SLICES", slices)
        with G.MeshGpt(0, config, 7, max_batch=96) as model:
            tokens = model.generate_tokens(prompts, 24, temperature, 7)
            results[slices] = (tokens, model.last_logits(96))
    for slices in ("2", "3"):
        assert np.array_equal(results[slices][0], results["1"][0]), f"{slices} slices: tokens differ"
        assert np.array_equal(results[slices][1], results["1"][1]), f"{slices} slices: logits differ"


def test_decode_slices_with_their_own_split_counts(monkeypatch):
    # 97 sequences in three slices of 32, 32 and 33: the first two split each
    # head's keys in two, the third and the whole batch do not, so the
    # slices' attention partial states sit at uneven offsets.  Greedy tokens
    # against one stream (up to near-ties) and final logits within TOL.
    config = G.named_config("mid")
    monkeypatch.setenv("MG_DISABLE_PERSISTENT", "1")
    monkeypatch.setenv("MG_ROW_BATCH", "1")
    prompts = G.random_prompts(256, 97, 16, 7)
    monkeypatch.setenv("MG_DECODE_SLICES", "1")
    with G.MeshGpt(0, config, 7, max_batch=97) as model:
        one = model.generate_tokens(prompts, 24, 0.0, 7)
        one_logits = model.last_logits(97)
    monkeypatch.setenv("MG_DECODE_SLICES", "3")
    with G.MeshGpt(0, config, 7, max_batch=97) as model:
        three = model.generate_tokens(prompts, 24, 0.0, 7)
        compared = assert_same_tokens_or_near_tie(model, three, one, "three slices")
        assert compared > 0.99 * three.size
        if np.array_equal(three, one):
            assert_close(model.last_logits(97), one_logits, what="three slices: final logits")


@pytest.mark.parametrize("name,batch", [("mid", 99), ("high", 23)])
def test_row_batches_match_single_rows(name, batch, monkeypatch):
    # The per-phase row blocks with 2 or 4 rows per workgroup (the last
    # workgroup's spare rows repeat the batch's last row and write nothing:
    # 99 and 23 rows leave 1 and 3 of them) against one row per workgroup:
    # greedy tokens up to near-ties, and the final logits within TOL; then
    # the 4-row run's logits against the oracle on its own tokens.
    config = G.named_config(name)
    monkeypatch.setenv("MG_DISABLE_PERSISTENT", "1")
    monkeypatch.setenv("MG_DECODE_SLICES", "1")
    prompts = G.random_prompts(256, batch, 16, 7)
    runs = {}
    for rb in ("1", "2", "4"):
        monkeypatch.setenv("MG_ROW_BATCH", rb)
        with G.MeshGpt(0, config, 7, max_batch=batch) as model:
            tokens = model.generate_tokens(prompts, 12, 0.0, 7)
            runs[rb] = (tokens, model.last_logits(batch))
            if rb == "1":
                continue
            compared = assert_same_tokens_or_near_tie(model, tokens, runs["1"][0], f"{rb} rows per workgroup")
            assert compared > 0.99 * tokens.size
            same = np.all(tokens == runs["1"][0], axis=1)
            assert_close(runs[rb][1][same], runs["1"][1][same], what=f"{rb} rows per workgroup: final logits")
    o = oracle_config(config)
    params = O.initialize(o, 7)
    tokens, last = runs["4"]
    for b in (0, batch - 1):
        ref = O.logits(o, params, tokens[b, :-1], tokens.shape[1] - 1)[-1]
        assert_close(last[b], ref, what=f"{name} 4 rows per workgroup, sequence {b}")


def test_cli_init_then_generate_matches_oracle(tmp_path):
    # `mesh-gpt init` writes the seeded default model with the demo corpus's
    # tokenizer; `mesh-gpt generate` (src/bin/mesh-gpt.rs:149-164) prints
    # decode(prompt + generated).  Greedy output must be the oracle's tokens;
    # the default T=0.7 output must pass the trajectory rule.  With context 32
    # and 240 tokens, most steps slide the window.
    cli = G.CLI_PATH
    checkpoint = str(tmp_path / "model.bin")
    corpus = os.path.join(ROOT, "tests", "golden", "mesh-gpt-demo.txt")
    res = subprocess.run([cli, "init", "--dataset", corpus, "--checkpoint", checkpoint],
                         capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    saved = G.Checkpoint.load(checkpoint)
    tokenizer = G.CharacterTokenizer(saved.characters)
    g = saved.config
    o = oracle_config(g)
    params = O.initialize(o, 7)
    assert np.array_equal(saved.parameters.view(np.uint32), params.view(np.uint32))
    prompt = "the little robot "
    ids = np.array(tokenizer.encode(prompt), dtype=np.uint32)
    for temperature in ("0", None):
        args = [cli, "generate", "--checkpoint", checkpoint]
        if temperature is not None:
            args += ["--temperature", temperature]
        res = subprocess.run(args, capture_output=True, text=True, timeout=120)
        assert res.returncode == 0, res.stderr
        assert res.stdout.endswith("\n")
        text = res.stdout[:-1]
        assert text.startswith(prompt)
        got = np.array(tokenizer.encode(text), dtype=np.uint32)
        assert got.size == ids.size + 240
        T = 0.0 if temperature == "0" else 0.7
        with G.MeshGpt(0, g, 7) as model:
            model.set_parameters(saved.parameters)
            check_trajectory(o, params, ids, got, T, 7, last_row_logits(model), cached=False)


def test_cli_prompt_file_and_normal_init(tmp_path):
    # generate --prompt-file: with --batch, one prompt per line (equal token
    # lengths), sequence b sampled with seed + b; without, the whole file is the
    # prompt, as --prompt.  generate --config tiny --init normal: the N(0, 0.5)
    # model.  Each output against the oracle's trajectory.
    cli = G.CLI_PATH
    checkpoint = str(tmp_path / "model.bin")
    corpus = os.path.join(ROOT, "tests", "golden", "mesh-gpt-demo.txt")
    res = subprocess.run([cli, "init", "--dataset", corpus, "--checkpoint", checkpoint],
                         capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    saved = G.Checkpoint.load(checkpoint)
    tokenizer = G.CharacterTokenizer(saved.characters)
    o = oracle_config(saved.config)
    params = O.initialize(o, 7)
    lines = ["the little robot ", "a quiet dog sang "]
    batch_file, one_file = tmp_path / "prompts.txt", tmp_path / "prompt.txt"
    batch_file.write_text("\n".join(lines) + "\n")
    one_file.write_text(lines[1])
    with G.MeshGpt(0, saved.config, 7) as model:
        model.set_parameters(saved.parameters)
        for path, extra, texts in ((batch_file, ["--batch", "2"], lines), (one_file, [], lines[1:])):
            res = subprocess.run([cli, "generate", "--checkpoint", checkpoint, "--prompt-file", str(path),
                                  "--tokens", "24", "--temperature", "0.8"] + extra,
                                 capture_output=True, text=True, timeout=120)
            assert res.returncode == 0, res.stderr
            # Each sequence prints its prompt and 24 generated characters (one
            # a token; the corpus has a newline character), then a newline.
            outs, at = [], 0
            for text in texts:
                n = len(text) + 24
                outs.append(res.stdout[at:at + n])
                assert res.stdout[at + n] == "\n"
                at += n + 1
            assert at == len(res.stdout)
            for b, (text, out) in enumerate(zip(texts, outs)):
                assert out.startswith(text)
                ids = np.array(tokenizer.encode(text), dtype=np.uint32)
                got = np.array(tokenizer.encode(out), dtype=np.uint32)
                check_trajectory(o, params, ids, got, 0.8, 7 + b, last_row_logits(model), cached=False)
    bad = tmp_path / "bad.txt"
    bad.write_text("the little robot \nshort\n")
    res = subprocess.run([cli, "generate", "--checkpoint", checkpoint, "--prompt-file", str(bad), "--batch", "2"],
                         capture_output=True, text=True, timeout=60)
    assert res.returncode == 1 and "batched prompts must have equal token lengths" in res.stderr
    res = subprocess.run([cli, "generate", "--checkpoint", checkpoint, "--prompt-file", str(bad), "--batch", "3"],
                         capture_output=True, text=True, timeout=60)
    assert res.returncode == 1 and "prompt file must hold one line per sequence (3), found 2" in res.stderr
    # A synthetic model with N(0, 0.5) weights and a seeded random prompt,
    # decoded first by this process with the persistent kernel, then by the
    # CLI (a second process on the same GPU, with its own persistent
    # launch): the same tokens.
    tiny = G.named_config("tiny")
    ot = oracle_config(tiny)
    prompt = G.random_prompts(64, 1, 16, 7)[0]
    weights = O.initialize_normal(ot, 7, 0.5)
    with G.MeshGpt(0, tiny, 7) as model:
        model.set_parameters(weights)
        here = model.generate_tokens(prompt[None, :], 32, 0.0, 7)[0]
        res = subprocess.run([cli, "generate", "--config", "tiny", "--init", "normal", "--random-prompt", "16",
                              "--batch", "1", "--tokens", "32", "--temperature", "0"],
                             capture_output=True, text=True, timeout=120)
        assert res.returncode == 0, res.stderr
        chars = [0x20 + i for i in range(64)]
        got = np.array([chars.index(ord(ch)) for ch in res.stdout[:-1]], dtype=np.uint32)
        assert np.array_equal(got, here)
        check_trajectory(ot, weights, prompt, got, 0.0, 7, last_row_logits(model))


MFMA_SHAPES = [
    dict(vocab_size=64, width=128, heads=4, layers=2, attention_mesh_depth=7, ffn_mesh_depth=7, context=512,
         connectivity=1),
    dict(vocab_size=256, width=512, heads=8, layers=2, attention_mesh_depth=9, ffn_mesh_depth=9, context=512,
         connectivity=1),
]


@pytest.mark.parametrize("cfg", MFMA_SHAPES, ids=["hd32", "hd64"])
def test_matrix_core_prefill_matches_oracle_and_valu(cfg, monkeypatch):
    # Prefill attention on the FP32 matrix cores (with XSA in its epilogue)
    # against the oracle's logits for every row, and against the VALU flash
    # kernel, over sequence lengths around its 16-query blocks, 64-key tiles
    # and 128-query workgroups.
    g = G.GptConfig(**cfg)
    o = oracle_config(g)
    params = O.initialize(o, 7)
    for n, batch in ((64, 2), (127, 1), (129, 2), (300, 1), (512, 1)):
        x = G.random_prompts(cfg["vocab_size"], batch, n, n).reshape(-1)
        got = {}
        for disable in ("0", "1"):
            monkeypatch.setenv("MG_DISABLE_MFMA_PREFILL", disable)
            with G.MeshGpt(0, g, 7) as model:
                got[disable] = model.logits(x, n)
        assert_close(got["0"], got["1"], what=f"matrix-core vs VALU prefill n={n}")
        ref = O.logits(o, params, x, n)
        assert_close(got["0"], ref, what=f"matrix-core prefill vs oracle n={n}")


ROWS_SHAPES = [
    dict(vocab_size=99, width=128, heads=4, layers=2, attention_mesh_depth=4, ffn_mesh_depth=6, context=80),
    dict(vocab_size=64, width=256, heads=8, layers=2, attention_mesh_depth=5, ffn_mesh_depth=3, context=80,
         connectivity=1),
    dict(vocab_size=256, width=512, heads=16, layers=2, attention_mesh_depth=9, ffn_mesh_depth=9, context=80,
         connectivity=1),
    dict(vocab_size=256, width=1024, heads=16, layers=2, attention_mesh_depth=10, ffn_mesh_depth=10, context=80,
         connectivity=1, embedding=1),
]


@pytest.mark.parametrize("cfg", ROWS_SHAPES, ids=["W128-hd32", "W256-hd32", "W512-hd32", "W1024-hd64-table"])
def test_register_tile_prefill_matches_oracle_and_block_kernel(cfg, monkeypatch):
    # The register-tile prefill block kernel (prefill_rows.hip) against the
    # oracle's logits and hidden states for every row, and against
    # block_kernel, with row counts that leave partial tiles; short sequences
    # take the VALU attention (XSA in the block's post half), 70-row ones the
    # matrix-core attention (XSA in its epilogue).
    g = G.GptConfig(**cfg)
    o = oracle_config(g)
    params = O.initialize(o, 7)
    for n, batch in ((4, 9), (7, 3), (70, 3)):
        x = G.random_prompts(cfg["vocab_size"], batch, n, n).reshape(-1)
        got = {}
        for disable in ("0", "1"):
            monkeypatch.setenv("MG_DISABLE_ROWS_PREFILL", disable)
            with G.MeshGpt(0, g, 7) as model:
                got[disable] = (model.logits(x, n), model.hidden_states(x, n))
        ref = O.logits(o, params, x, n)
        assert_close(got["0"][0], ref, what=f"register-tile prefill logits n={n}")
        assert_close(got["0"][1], O.hidden_states(o, params, x, n), what=f"register-tile hidden n={n}")
        assert_close(got["0"][0], got["1"][0], what=f"register-tile vs block_kernel n={n}")
