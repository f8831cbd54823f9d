"""GPU parity: the HIP path through the C ABI against the f64 CPU oracle.

Mirrors the reference's GPU verification (src/bin/mesh-gpt.rs:324-553, the
config list at 651-857): seeded weights (seed 7), inputs x[i] = i % V, every
logit within TOL*(1+|ref|), effective embeddings, causality and prefix checks,
and the rejection cases.  Generation is checked token by token against the
oracle's generate loop (src/gpt/gpu.rs:2006-2053).
"""
import numpy as np
import pytest

import grokking_abmod_amd as G
import oracle_lib as O
from conftest import TOL, assert_close
from trajectory import check_trajectory

pytestmark = pytest.mark.gpu


def configs_for(**kw):
    """The same GptConfig for the product (mg_config) and the oracle (og_config)."""
    g = G.GptConfig(**kw)
    o = O.config(**{k: v for k, v in kw.items() if k != "long_context"})
    return g, o


# (config, cases) from src/bin/mesh-gpt.rs:651-857 (geometry ablations excluded).
VERIFY = [
    (dict(vocab_size=129, context=3, width=2, heads=1, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (1, 3), (2, 3), (43, 3)]),
    (dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (1, 3), (2, 3), (43, 3)]),
    (dict(vocab_size=7, context=5, width=8, heads=2, layers=2, attention_mesh_depth=3, ffn_mesh_depth=4),
     [(1, 1), (1, 3), (2, 3), (43, 3)]),
    (dict(vocab_size=9, context=3, width=64, heads=8, layers=1, attention_mesh_depth=1, ffn_mesh_depth=1),
     [(1, 1), (1, 3), (2, 3), (43, 3)]),
    (dict(vocab_size=9, context=3, width=128, heads=4, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (1, 3), (2, 3), (43, 3)]),
    (dict(vocab_size=5, context=5, width=4, heads=2, layers=3, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (2, 3), (43, 3)]),
    (dict(vocab_size=11, context=5, width=6, heads=3, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (2, 3), (43, 3)]),
    (dict(vocab_size=257, context=129, width=256, heads=16, layers=3, attention_mesh_depth=2,
          ffn_mesh_depth=2), [(1, 1), (1, 3), (2, 3)]),
    (dict(vocab_size=5, context=129, width=4, heads=2, layers=1, attention_mesh_depth=1, ffn_mesh_depth=1),
     [(1, 129)]),
    (dict(vocab_size=7, context=3, width=1024, heads=4, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (1, 3), (2, 3)]),
    (dict(vocab_size=99, context=4, width=32, heads=4, layers=1, attention_mesh_depth=1, ffn_mesh_depth=1),
     [(1, 1), (1, 4), (2, 4)]),
    (dict(vocab_size=99, context=4, width=32, heads=4, layers=1, attention_mesh_depth=5, ffn_mesh_depth=6,
          embedding=1, connectivity=1), [(1, 1), (1, 4), (2, 4), (33, 4)]),
] + [
    (dict(base, embedding=e, connectivity=k), cases)
    for e, k in ((1, 0), (0, 1), (1, 1))
    for base, cases in (
        (dict(vocab_size=7, context=5, width=8, heads=2, layers=2, attention_mesh_depth=3, ffn_mesh_depth=4),
         [(1, 1), (1, 3), (2, 3), (43, 3)]),
        (dict(vocab_size=9, context=3, width=128, heads=4, layers=1, attention_mesh_depth=8,
              ffn_mesh_depth=8), [(1, 1), (1, 3), (2, 3), (43, 3)]),
    )
] + [
    (dict(vocab_size=5, context=129, width=w, heads=h, layers=1, attention_mesh_depth=1, ffn_mesh_depth=1),
     [(1, 33), (1, 129), (2, 33)])
    for w, h in ((32, 1), (64, 2), (64, 1))
]


def _ids(cfg):
    return "V{vocab_size}-W{width}-H{heads}-L{layers}-A{attention_mesh_depth}-F{ffn_mesh_depth}".format(**cfg) + \
        ("-table" if cfg.get("embedding") else "") + ("-butterfly" if cfg.get("connectivity") else "")


@pytest.mark.parametrize("cfg,cases", VERIFY, ids=[_ids(c) for c, _ in VERIFY])
def test_verify_model_logits(cfg, cases):
    g, o = configs_for(**cfg)
    params = O.initialize(o, 7)
    with G.MeshGpt(0, g, 7) as model:
        # The product seeds the same weights as the oracle's restatement.
        assert np.array_equal(model.parameters().view(np.uint32), params.view(np.uint32))
        assert_close(model.token_embeddings(), O.token_embeddings(o, params), what="embeddings")
        for batch, sequence in cases:
            x = (np.arange(batch * sequence) % cfg["vocab_size"]).astype(np.uint32)
            expected = O.logits(o, params, x, sequence)
            actual = model.logits(x, sequence)
            assert_close(actual, expected, what=f"logits batch={batch} sequence={sequence}")
            last = model.logits(x, sequence, last_only=True)
            assert_close(last, expected.reshape(batch, sequence, -1)[:, -1], what="last-row logits")
            hidden = model.hidden_states(x, sequence)
            assert_close(hidden, O.hidden_states(o, params, x, sequence), what="hidden states")
        if cfg["context"] >= 3 and cfg["vocab_size"] >= 5:
            # Causal mask and prefix invariance (mesh-gpt.rs:387-394).
            full = model.logits([0, 1, 2], 3)
            changed = model.logits([0, 1, 4], 3)
            assert np.array_equal(full[:2], changed[:2])
            assert np.array_equal(full[:2], model.logits([0, 1], 2))


def test_verify_command_quick_run():
    # tests/verify.py, this build's `mesh-gpt verify` (mesh-gpt.rs:624-896),
    # on its first three models and one geometry: one PASS line each, exit 0.
    import subprocess
    import sys

    here = __import__("os").path.dirname(__import__("os").path.abspath(__file__))
    res = subprocess.run([sys.executable, __import__("os").path.join(here, "verify.py"), "--quick"],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.splitlines()
    assert len(lines) == 4 and all(line.startswith("PASS ") for line in lines), res.stdout
    assert "AdamW beta2=0.999/0.98/reset, zero-weight behavior" in lines[0]


def test_rejections_match_reference_messages():
    g, o = configs_for(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2,
                       ffn_mesh_depth=2)
    with G.MeshGpt(0, g, 7) as model:
        shape_msg = "tokens must form a nonempty batch of equal sequences within context and 131072 rows"
        for tokens, sequence, message in (
            ([], 1, shape_msg),
            ([2**32 - 1], 1, "token ID is outside the vocabulary"),
            ([0], 0, shape_msg),
            ([0, 1, 2], 2, shape_msg),
            ([0] * 5, 5, shape_msg),
        ):
            with pytest.raises(G.MeshGptError, match=message):
                model.logits(tokens, sequence)
        with pytest.raises(G.MeshGptError, match="parameter count does not match GPT configuration"):
            model.set_parameters([0.0])
        bad = O.initialize(o, 7)
        bad[3] = np.nan
        with pytest.raises(G.MeshGptError, match="parameters must contain only finite values"):
            model.set_parameters(bad)
        with pytest.raises(G.MeshGptError, match=r"temperature must be finite and nonnegative \(0 is greedy\)"):
            model.generate_tokens([[0, 1]], 3, -1.0, 7)
        with pytest.raises(G.MeshGptError, match=r"temperature must be finite and nonnegative"):
            model.generate_tokens([[0, 1]], 3, float("nan"), 7)
        with pytest.raises(G.MeshGptError, match="tokenizer does not match model vocabulary size"):
            model.generate("abc", "ab", 3, 0.0, 7)
        with pytest.raises(G.MeshGptError, match="generation prompt must not be empty"):
            model.generate("abcde", "", 3, 0.0, 7)
        with pytest.raises(G.MeshGptError, match="character 'z' is outside the tokenizer vocabulary"):
            model.generate("abcde", "az", 3, 0.0, 7)


def test_zero_embedding_gives_zero_logits():
    # reference.rs:838-861 on the device path.
    for emb in (0, 1):
        for conn in (0, 1):
            g, o = configs_for(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2,
                               ffn_mesh_depth=2, embedding=emb, connectivity=conn)
            params = np.full(O.parameter_count(o), 0.5, dtype=np.float32)
            params[:O.lib().og_embedding_parameter_count(o)] = 0.0
            with G.MeshGpt(0, g, 7) as model:
                model.set_parameters(params)
                assert np.array_equal(model.logits([0, 1, 2, 3, 4, 0], 3), np.zeros((6, 5), np.float32))


def _overflowing_v_mesh(o, params):
    """Block 0's V mesh with every weight 3e38: its rows overflow to +inf in f32
    (and, after 8 ELU layers of growth by 6e38, in the f64 oracle too).  XSA
    then divides inf by inf, so every head's output is NaN, and the projection
    mesh's ELU layers must carry the NaN on (reference.rs:325-332: NaN >= 0 is
    false and exp_m1(NaN) is NaN) so that the logits are non-finite."""
    bad = params.copy()
    start = O.group_offsets(o)[1 + 2]  # embedding mesh, then block 0's q, k, v
    size = 2 * o.width * o.attention_mesh_depth
    bad[start:start + size] = 3e38
    return bad


@pytest.mark.parametrize("shape", ["W512-A9", "W128-A9-short"])
def test_nan_inside_a_mesh_reaches_the_logits(shape, monkeypatch):
    """A NaN born inside the model (inf / inf in XSA) must make the logits
    non-finite on every path, prefill (register-tile and short-sequence
    kernels), the persistent decode and the per-phase decode, so that the
    calls return MG_NONFINITE as the reference's "logits must contain only
    finite values" (gpu.rs:1903-1913).  The f64 oracle's logits are non-finite
    for the same weights."""
    if shape == "W512-A9":
        kw = dict(vocab_size=256, context=128, width=512, heads=8, layers=2, attention_mesh_depth=9,
                  ffn_mesh_depth=9, connectivity=1)
        n = 64
    else:
        kw = dict(vocab_size=64, context=64, width=128, heads=4, layers=2, attention_mesh_depth=9,
                  ffn_mesh_depth=9, connectivity=1)
        n = 8
    g, o = configs_for(**kw)
    bad = _overflowing_v_mesh(o, O.initialize(o, 7))
    tokens = G.random_prompts(kw["vocab_size"], 2, n, 7)
    assert not np.isfinite(O.logits(o, bad, tokens[0], n)).all()
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_PERSISTENT", disable)
        with G.MeshGpt(0, g, 7, max_batch=2) as model:
            model.set_parameters(bad)
            for last_only in (False, True):
                with pytest.raises(G.MeshGptError, match="logits must contain only finite values") as err:
                    model.logits(tokens.reshape(-1), n, last_only=last_only)
                assert err.value.status == G.MG_NONFINITE
            with pytest.raises(G.MeshGptError) as err:
                model.generate_tokens(tokens, 4, 0.0, 7)
            assert err.value.status == G.MG_NONFINITE, str(err.value)


def _device_last(model):
    return lambda window: model.logits(window, len(window), last_only=True)[0]


def test_generate_greedy_tiny_config1():
    # V64 W128 H4x32 L2 butterfly depth 7, ctx 256, 16-token prompt, 128 greedy.
    g, o = configs_for(vocab_size=64, context=256, width=128, heads=4, layers=2, attention_mesh_depth=7,
                       ffn_mesh_depth=7, connectivity=1)
    params = O.initialize(o, 7)
    prompt = G.random_prompts(64, 1, 16, 7)[0]
    with G.MeshGpt(0, g, 7) as model:
        got = model.generate_tokens(prompt[None, :], 128, 0.0, 7)[0]
        check_trajectory(o, params, prompt, got, 0.0, 7, _device_last(model))
        # The last step's logits equal a full re-prefill of the same tokens on the device.
        full = model.logits(got[:-1], len(got) - 1, last_only=True)
        assert_close(model.last_logits(1), full, what="KV decode vs re-prefill")


def test_kv_cache_decode_equals_reference_recompute():
    # The oracle's reference-semantics loop (full window recompute each token)
    # and its KV-cached loop agree exactly; the device decode must match both.
    g, o = configs_for(vocab_size=11, context=24, width=16, heads=2, layers=2, attention_mesh_depth=3,
                       ffn_mesh_depth=4)
    params = O.initialize(o, 3)
    prompt = np.array([1, 4, 2, 9, 0], dtype=np.uint32)
    ref = O.generate(o, params, prompt, 19, 0.0, 5)
    assert np.array_equal(ref, O.generate(o, params, prompt, 19, 0.0, 5, cached=True))
    with G.MeshGpt(0, g, 3) as model:
        got = model.generate_tokens(prompt[None, :], 19, 0.0, 5)[0]
        check_trajectory(o, params, prompt, got, 0.0, 5, _device_last(model), expected=ref)


def test_sliding_window_beyond_context_matches_reference():
    # gpu.rs:2026: once the sequence is longer than the context the window
    # slides and positions restart at 0 every step.
    g, o = configs_for(vocab_size=7, context=6, width=8, heads=2, layers=2, attention_mesh_depth=3,
                       ffn_mesh_depth=4, connectivity=1)
    params = O.initialize(o, 11)
    prompt = np.array([3, 1, 4], dtype=np.uint32)
    for temperature in (0.0, 0.9):
        with G.MeshGpt(0, g, 11) as model:
            got = model.generate_tokens(prompt[None, :], 25, temperature, 13)[0]
            check_trajectory(o, params, prompt, got, temperature, 13, _device_last(model), cached=False)


def test_batch_rows_equal_single_sequences():
    # Row b of a batched generate is the B=1 generate with seed + b, bit for bit.
    g, o = configs_for(vocab_size=64, context=64, width=128, heads=4, layers=2, attention_mesh_depth=7,
                       ffn_mesh_depth=7, connectivity=1)
    prompts = (np.arange(5 * 8).reshape(5, 8) * 7 % 64).astype(np.uint32)
    with G.MeshGpt(0, g, 7, max_batch=5) as model:
        batched = model.generate_tokens(prompts, 40, 0.8, 100)
        for b in range(5):
            single = model.generate_tokens(prompts[b:b + 1], 40, 0.8, 100 + b)[0]
            assert np.array_equal(batched[b], single), f"row {b}"


def test_temperature_sampling_matches_oracle():
    g, o = configs_for(vocab_size=64, context=128, width=128, heads=4, layers=2, attention_mesh_depth=7,
                       ffn_mesh_depth=7, connectivity=1)
    params = O.initialize(o, 7)
    prompt = (np.arange(16) * 5 % 64).astype(np.uint32)
    temperature = 0.7
    with G.MeshGpt(0, g, 7) as model:
        got = model.generate_tokens(prompt[None, :], 96, temperature, 21)[0]
        check_trajectory(o, params, prompt, got, temperature, 21, _device_last(model))


def test_symbolic_config2_published_cross_entropy():
    # BASELINE config 2 = grok defaults (mod 97 add, seed 7, W128 H4 L2 A4 F6,
    # neighbor): one prefill of all 9409 equations, last-position logits.  The
    # mean cross-entropies over the two splits were published from the
    # reference's CUDA path (docs/cuda-performance.md:238-240), and answer
    # accuracy was zero at that point (docs/grokking.md:179-180).  Each row's
    # prediction (row_metrics: first maximal logit, grokking.rs(bin):544-586)
    # equals the oracle's wherever the top-2 gap exceeds the logit tolerance.
    g, o = configs_for(vocab_size=99, context=4, width=128)
    params = O.initialize(o, 7)
    res, train, valid = O.equations()
    with G.MeshGpt(0, g, 7) as model:
        for eqs, published in ((train, 7.419670094), (valid, 7.432581042)):
            x, targets = O.equation_inputs(res, eqs)
            logits = model.logits(x, 4, last_only=True)
            metrics = [O.row_metrics(row, int(t)) for row, t in zip(logits, targets)]
            ce = np.mean([m[0] for m in metrics])
            assert abs(ce - published) < 2e-6, ce
            predicted = np.array([m[1] for m in metrics])
            assert np.mean(predicted == targets) == 0.0
            ref = O.logits(o, params, x, 4).reshape(-1, 4, 99)[:, -1]
            assert_close(logits, ref, what="config-2 logits")
            top2 = np.sort(ref, axis=1)[:, -2:]
            clear = top2[:, 1] - top2[:, 0] > 2 * TOL * (1 + np.abs(top2[:, 1]))
            assert np.array_equal(predicted[clear], np.argmax(ref, axis=1)[clear])


def test_mid_config3_decode_parity_subset():
    # BASELINE config 3 shapes (V256 W512 H8x64 L6 butterfly depth 9, ctx 1024,
    # T=1.0 seeded): 4 of the 32 sequences, 64-token prompts, 48 decode steps.
    g, o = configs_for(vocab_size=256, context=1024, width=512, heads=8, layers=6, attention_mesh_depth=9,
                       ffn_mesh_depth=9, connectivity=1)
    params = O.initialize(o, 7)
    prompts = G.random_prompts(256, 4, 64, 3)
    with G.MeshGpt(0, g, 7, max_batch=4) as model:
        got = model.generate_tokens(prompts, 48, 1.0, 7)
        for b in range(4):
            check_trajectory(o, params, prompts[b], got[b], 1.0, 7 + b, _device_last(model))
        # Decode logits at the last step equal the oracle's on the device's own tokens.
        last = model.last_logits(4)
        for b in range(2):
            ref = O.logits(o, params, got[b, :-1], got.shape[1] - 1)[-1]
            assert_close(last[b], ref, what=f"config-3 logits seq {b}")


# Decode shapes that exercise each row-order kernel instantiation: the
# fixed-depth ones of the benchmark configs above, and the any-depth form for
# neighbor meshes (every layer crosses waves), head groups of 8 and 32 lanes,
# and widths 256 and 1024.
ROW_DECODE = [
    dict(vocab_size=64, context=32, width=128, heads=4, layers=2, attention_mesh_depth=3, ffn_mesh_depth=5),
    dict(vocab_size=32, context=32, width=256, heads=8, layers=1, attention_mesh_depth=4, ffn_mesh_depth=4,
         connectivity=1),
    dict(vocab_size=32, context=32, width=512, heads=4, layers=2, attention_mesh_depth=9, ffn_mesh_depth=8,
         connectivity=1),
    dict(vocab_size=16, context=16, width=1024, heads=16, layers=1, attention_mesh_depth=2, ffn_mesh_depth=3,
         connectivity=1),
    dict(vocab_size=16, context=16, width=1024, heads=16, layers=1, attention_mesh_depth=10, ffn_mesh_depth=10,
         connectivity=1),
]


@pytest.mark.parametrize("cfg", ROW_DECODE, ids=[_ids(c) for c in ROW_DECODE])
def test_row_decode_shapes_match_oracle(cfg):
    g, o = configs_for(**cfg)
    params = O.initialize(o, 5)
    prompts = (np.arange(2 * 5).reshape(2, 5) * 3 % cfg["vocab_size"]).astype(np.uint32)
    with G.MeshGpt(0, g, 5, max_batch=2) as model:
        got = model.generate_tokens(prompts, 6, 0.0, 9)
        last = model.last_logits(2)
        for b in range(2):
            ref = O.logits(o, params, got[b, :-1], got.shape[1] - 1)[-1]
            assert_close(last[b], ref, what=f"decode logits seq {b}")
            check_trajectory(o, params, prompts[b], got[b], 0.0, 9 + b, _device_last(model))


@pytest.mark.parametrize("name", ["tiny", "mid"])
def test_decode_kernels_agree(name, monkeypatch):
    # The row-order decode kernel and the one-wave-per-mesh kernel decode the
    # same tokens, with last-step logits within the tolerance of each other.
    config = G.named_config(name)
    prompts = (np.arange(4 * 24).reshape(4, 24) * 7 % config.vocab_size).astype(np.uint32)
    results = []
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_ROW_DECODE", disable)
        with G.MeshGpt(0, config, 7, max_batch=4) as model:
            tokens = model.generate_tokens(prompts, 24, 0.0, 7)
            results.append((tokens, model.last_logits(4)))
    (t0, l0), (t1, l1) = results
    assert np.array_equal(t0, t1)
    assert_close(l0, l1, what="row vs wave decode logits")


@pytest.mark.parametrize("name,temperature", [("tiny", 0.0), ("tiny", 0.8), ("mid", 0.0), ("mid", 1.0)])
def test_persistent_decode_matches_per_phase_kernels(name, temperature, monkeypatch):
    # The persistent decode launch (all steps in one kernel) and the per-phase
    # kernels decode the same tokens from the same prompts and seeds, with
    # last-step logits within the tolerance of each other.
    config = G.named_config(name)
    prompts = (np.arange(6 * 20).reshape(6, 20) * 5 % config.vocab_size).astype(np.uint32)
    results = []
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_PERSISTENT", disable)
        with G.MeshGpt(0, config, 7, max_batch=6) as model:
            tokens = model.generate_tokens(prompts, 40, temperature, 11)
            results.append((tokens, model.last_logits(6)))
    (t0, l0), (t1, l1) = results
    assert np.array_equal(t0, t1)
    assert_close(l0, l1, what="persistent vs per-phase decode logits")


def test_persistent_decode_timeout_falls_back_to_per_phase_kernels(monkeypatch):
    # A persistent launch whose hand-off waits time out (forced from the host
    # with a wait limit of one 100 MHz tick, so a wait that has to poll gives
    # up at its first unanswered poll) ends with its abort flag set; the library then
    # restores the decode state and runs the same steps on the per-phase
    # kernels, so tokens and last-step logits equal a per-phase run's bit for
    # bit.  With MG_PERSIST_STRICT=1 the same launch raises a device error.
    config = G.named_config("mid")
    prompts = G.random_prompts(256, 8, 20, 7)
    runs = []
    for env in ({"MG_DISABLE_PERSISTENT": "1"},
                {"MG_PERSIST_WAIT_TICKS": "1", "MG_PERSIST_STRICT": "0", "MG_FORCE_PERSISTENT": "1"}):
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        with G.MeshGpt(0, config, 7, max_batch=8) as model:
            model.prefill(prompts, 1.0, 11, reserve=20 + 1 + 16)
            model.decode(16)
            assert model.sequence_length() == 20 + 1 + 16
            runs.append((model.read_tokens(8), model.last_logits(8)))
        for k in env:
            monkeypatch.delenv(k)
    assert np.array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1], runs[1][1])
    # Strict: the timed-out launch raises and leaves the decode state as it
    # was, so the same steps then decode (with the default wait limit) to
    # what a fresh model decodes.
    monkeypatch.setenv("MG_PERSIST_STRICT", "1")
    monkeypatch.setenv("MG_FORCE_PERSISTENT", "1")
    with G.MeshGpt(0, config, 7, max_batch=8) as model:
        model.prefill(prompts, 1.0, 11, reserve=20 + 1 + 4)
        model.decode(4)
        fresh = model.read_tokens(8)
    with G.MeshGpt(0, config, 7, max_batch=8) as model:
        model.prefill(prompts, 1.0, 11, reserve=20 + 1 + 4)
        monkeypatch.setenv("MG_PERSIST_WAIT_TICKS", "1")
        with pytest.raises(G.MeshGptError, match="timed out waiting on a hand-off") as err:
            model.decode(4)
        assert err.value.status == G.MG_DEVICE_ERROR
        assert model.sequence_length() == 20 + 1
        monkeypatch.delenv("MG_PERSIST_WAIT_TICKS")
        model.decode(4)
        assert np.array_equal(model.read_tokens(8), fresh)


def test_persistent_decode_full_batch_matches_per_phase_kernels(monkeypatch):
    # 32 sequences of config 3 need more workgroups than the GPU has CUs, so
    # some share a CU and the launch maps roles to workgroups with its pairing
    # map; it must decode what the per-phase kernels decode.
    config = G.named_config("mid")
    prompts = (np.arange(32 * 20).reshape(32, 20) * 5 % config.vocab_size).astype(np.uint32)
    results = []
    for disable in ("0", "1"):
        monkeypatch.setenv("MG_DISABLE_PERSISTENT", disable)
        with G.MeshGpt(0, config, 7, max_batch=32) as model:
            tokens = model.generate_tokens(prompts, 24, 1.0, 13)
            results.append((tokens, model.last_logits(32)))
    (t0, l0), (t1, l1) = results
    assert np.array_equal(t0, t1)
    assert_close(l0, l1, what="persistent vs per-phase decode logits, batch 32")


def test_persistent_decode_steps_continue_a_generation():
    # decode(k) after prefill appends exactly the tokens a single generate call
    # produces (the persistent launch picks up the sampler state and lengths).
    config = G.named_config("tiny")
    prompts = (np.arange(3 * 16).reshape(3, 16) * 11 % config.vocab_size).astype(np.uint32)
    with G.MeshGpt(0, config, 7, max_batch=3) as model:
        whole = model.generate_tokens(prompts, 33, 0.9, 5)
        model.prefill(prompts, 0.9, 5, reserve=16 + 33)
        model.decode(12)
        model.decode(20)
        assert model.sequence_length() == 16 + 33
        assert np.array_equal(model.read_tokens(3), whole)


# MSHGPT09 ablations (checkpoint.rs:146-168): operator switches
# (reference.rs:174-199) and embedding geometry (reference.rs:130-149,
# geometry.rs:238-325) on the prefill and decode paths.
ABLATION_BASE = dict(vocab_size=7, context=96, width=128, heads=4, layers=2, attention_mesh_depth=3,
                     ffn_mesh_depth=3, connectivity=1)
ABLATIONS = [
    dict(rope=0), dict(qk_norm=0), dict(xsa=0), dict(rope=0, qk_norm=0, xsa=0), dict(xsa=0, embedding=1),
    dict(form=9), dict(normalization=2), dict(preserve_features=3), dict(form=1, order=2, modulus=5, seed=17),
    dict(form=2, harmonics=3, embedding=1, normalization=1), dict(form=5, overlap=0.25, embedding=1, qk_norm=0),
    dict(width=12, heads=4, rope=0),
]


@pytest.mark.parametrize("kw", ABLATIONS, ids=[str(i) for i in range(len(ABLATIONS))])
def test_mshgpt09_ablations_match_oracle(kw):
    cfg = dict(ABLATION_BASE, **kw)
    g, o = configs_for(**cfg)
    params = O.initialize(o, 7)
    with G.MeshGpt(0, g, 7, max_batch=2) as model:
        assert np.array_equal(model.parameters().view(np.uint32), params.view(np.uint32))
        assert_close(model.token_embeddings(), O.token_embeddings(o, params), what="embeddings")
        for batch, n in ((5, 4), (2, 70)):
            x = G.random_prompts(7, batch, n, n).reshape(-1)
            assert_close(model.logits(x, n), O.logits(o, params, x, n), what=f"logits n={n}")
        prompts = G.random_prompts(7, 2, 8, 1)
        got = model.generate_tokens(prompts, 12, 0.0, 3)
        last = model.last_logits(2)
        for b in range(2):
            assert_close(last[b], O.logits(o, params, got[b, :-1], got.shape[1] - 1)[-1], what=f"decode seq {b}")
            check_trajectory(o, params, prompts[b], got[b], 0.0, 3 + b, _device_last(model))


# The one-launch forward of sequences of up to 16 rows (a workgroup holds 4, 2
# or 1 of them by length, and the count need not divide by it): lengths across
# those cases, ragged counts, head widths 2 to 128, both connectivities and
# embeddings, all-row and last-row logits, a vocabulary beyond the workgroup.
SHORT = [
    (dict(vocab_size=11, context=16, width=128, heads=1, layers=2, attention_mesh_depth=3, ffn_mesh_depth=2),
     (1, 4, 5, 8, 9, 16)),
    (dict(vocab_size=67, context=16, width=64, heads=1, layers=1, attention_mesh_depth=2, ffn_mesh_depth=3,
          connectivity=1), (2, 7, 12)),
    (dict(vocab_size=300, context=16, width=16, heads=8, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2,
          embedding=1), (3, 6, 16)),
    # width 128 with neighbour connectivity keeps channels interleaved (2 lane + j):
    # head widths 2, 4, 16 and 64 and the ablation switches there
    (dict(vocab_size=13, context=16, width=128, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
          qk_norm=0), (3, 6)),
    (dict(vocab_size=13, context=16, width=128, heads=32, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
          xsa=0), (4, 11)),
    (dict(vocab_size=13, context=16, width=128, heads=64, layers=1, attention_mesh_depth=1, ffn_mesh_depth=2),
     (2, 16)),
    (dict(vocab_size=13, context=16, width=128, heads=8, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2,
          rope=0), (4,)),
    # butterfly strides at widths 128 and 32 (lane exchanges, channel lane + 64 j)
    (dict(vocab_size=13, context=16, width=128, heads=4, layers=2, attention_mesh_depth=9, ffn_mesh_depth=3,
          connectivity=1), (1, 6, 13)),
    (dict(vocab_size=13, context=16, width=32, heads=2, layers=1, attention_mesh_depth=6, ffn_mesh_depth=2,
          connectivity=1, embedding=1), (4, 16)),
]


@pytest.mark.parametrize("cfg,lengths", SHORT, ids=[_ids(c) for c, _ in SHORT])
def test_short_sequence_forward_matches_oracle(cfg, lengths):
    g, o = configs_for(**cfg)
    params = O.initialize(o, 5)
    with G.MeshGpt(0, g, 5) as model:
        for n in lengths:
            for batch in (1, 3, 7):
                x = G.random_prompts(cfg["vocab_size"], batch, n, n + batch).reshape(-1)
                expected = O.logits(o, params, x, n)
                assert_close(model.logits(x, n), expected, what=f"logits batch={batch} n={n}")
                assert_close(model.logits(x, n, last_only=True), expected.reshape(batch, n, -1)[:, -1],
                             what=f"last-row logits batch={batch} n={n}")
