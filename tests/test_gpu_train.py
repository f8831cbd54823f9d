"""GPU parity of the training step (f4): loss, gradients and AdamW through the C ABI.

Mirrors the training half of the reference's GPU verification
(src/bin/mesh-gpt.rs:324-553): seeded weights (seed 7), x[i] = i % V,
y[i] = (i + 2) % V and the answer-only targets (the last row of each sequence),
loss and every gradient within TOL * (1 + |ref|) of the f64 tape oracle (the
reference allows 5e-4; TOL is 1e-4); then three AdamW steps under the two
optimizer settings it checks, each step's gradient against the oracle's on the
GPU's own weights and the update against the f32 AdamW applied to the GPU's
own gradient.  Rejections carry the reference's messages.
"""
import numpy as np
import pytest

import grokking_abmod_amd as G
import oracle_lib as O
from conftest import TOL, assert_close

pytestmark = pytest.mark.gpu

IGN = G.IGNORE_TARGET


def configs_for(**kw):
    return G.GptConfig(**kw), O.config(**kw)


# (config, cases) from src/bin/mesh-gpt.rs:651-857, the demo and grok training
# shapes, each operator switched off, and the frozen geometry.
TRAIN = [
    (dict(vocab_size=129, context=3, width=2, heads=1, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (2, 3), (43, 3)]),
    (dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (1, 3), (2, 3), (43, 3)]),
    (dict(vocab_size=7, context=5, width=8, heads=2, layers=2, attention_mesh_depth=3, ffn_mesh_depth=4),
     [(1, 3), (43, 3)]),
    (dict(vocab_size=9, context=3, width=64, heads=8, layers=1, attention_mesh_depth=1, ffn_mesh_depth=1),
     [(2, 3), (43, 3)]),
    (dict(vocab_size=9, context=3, width=128, heads=4, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(2, 3), (43, 3)]),
    (dict(vocab_size=11, context=5, width=6, heads=3, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(2, 3), (43, 3)]),
    (dict(vocab_size=257, context=129, width=256, heads=16, layers=3, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 3), (2, 3)]),
    (dict(vocab_size=5, context=129, width=4, heads=2, layers=1, attention_mesh_depth=1, ffn_mesh_depth=1),
     [(1, 129)]),
    (dict(vocab_size=99, context=4, width=32, heads=4, layers=1, attention_mesh_depth=5, ffn_mesh_depth=6,
          embedding=1, connectivity=1), [(2, 4), (33, 4)]),
    (dict(vocab_size=9, context=3, width=128, heads=4, layers=1, attention_mesh_depth=8, ffn_mesh_depth=8,
          connectivity=1), [(2, 3), (43, 3)]),
    (dict(vocab_size=7, context=3, width=1024, heads=4, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(1, 1), (1, 3), (2, 3)]),
    (dict(vocab_size=7, context=5, width=512, heads=1, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2),
     [(2, 5)]),
    # the demo training shape (docs/mesh-gpt.md:240-243) and the grok shape
    (dict(vocab_size=26, context=32, width=32, heads=4, layers=2), [(2, 32)]),
    (dict(vocab_size=99, context=4, width=128, heads=4, layers=2), [(32, 4)]),
    (dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
          rope=0), [(2, 3)]),
    (dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
          qk_norm=0), [(2, 3)]),
    (dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
          xsa=0), [(2, 3)]),
    (dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
          frozen=1), [(2, 3)]),
]


# MSHGPT09 ablations (the inference tests' list, tests/test_gpu_parity.py):
# operator switches and embedding geometry forms, normalisation and protected
# coordinates (reference.rs:130-149, geometry.rs:238-325).
ABLATION_BASE = dict(vocab_size=7, context=12, width=128, heads=4, layers=2, attention_mesh_depth=3,
                     ffn_mesh_depth=3, connectivity=1)
ABLATIONS = [
    dict(rope=0, qk_norm=0, xsa=0), dict(xsa=0, embedding=1), dict(form=9), dict(normalization=2),
    dict(preserve_features=3), dict(form=1, order=2, modulus=5, seed=17),
    dict(form=2, harmonics=3, embedding=1, normalization=1), dict(form=5, overlap=0.25, embedding=1, qk_norm=0),
    dict(width=12, heads=4, rope=0), dict(preserve_features=2, frozen=1),
]
TRAIN += [(dict(ABLATION_BASE, **kw), [(3, 12)]) for kw in ABLATIONS]


def _ids(cfg):
    extra = "".join(f"-{k}{v}" for k, v in cfg.items() if k in ("embedding", "connectivity", "rope", "qk_norm",
                                                                  "xsa", "frozen", "form", "normalization",
                                                                  "preserve_features", "order", "overlap"))
    full = dict(attention_mesh_depth=4, ffn_mesh_depth=6)  # GptConfig::default() depths
    full.update(cfg)
    return "V{vocab_size}-W{width}-H{heads}-L{layers}-A{attention_mesh_depth}-F{ffn_mesh_depth}".format(**full) + extra


def batch(V, b, s):
    x = np.arange(b * s) % V
    y = (np.arange(b * s) + 2) % V
    answer = np.where(np.arange(b * s) % s == s - 1, y, IGN)
    return x.astype(np.uint32), y.astype(np.uint32), answer.astype(np.uint32)


@pytest.mark.parametrize("cfg,cases", TRAIN, ids=[_ids(c) for c, _ in TRAIN])
def test_loss_and_gradients_match_the_oracle(cfg, cases):
    g, o = configs_for(**cfg)
    params = O.initialize(o, 7)
    with G.MeshGpt(0, g, 7) as model:
        for b, s in cases:
            x, y, answer = batch(cfg["vocab_size"], b, s)
            for targets in (y, answer):
                ref_loss, ref_grad = O.loss_and_gradient(o, params, x, targets, s)
                loss, grad = model.loss_and_gradient(x, targets, s)
                assert abs(loss - ref_loss) <= TOL * (1 + abs(ref_loss)), (b, s, loss, ref_loss)
                assert_close(grad, ref_grad, what=f"gradient b={b} s={s}")
                assert abs(model.cross_entropy(x, targets, s) - loss) <= 1e-6 * (1 + abs(loss))


# Stacks deeper than the 16 layers of one kernel launch, in the wave (width
# <= 128) and the LDS (wider) mesh kernels, both connectivities, the mesh
# embedding included.
DEEP = [
    dict(vocab_size=7, context=3, width=8, heads=2, layers=1, attention_mesh_depth=32, ffn_mesh_depth=20),
    dict(vocab_size=7, context=3, width=8, heads=2, layers=1, attention_mesh_depth=17, ffn_mesh_depth=33,
         embedding=1, connectivity=1),
    dict(vocab_size=7, context=3, width=128, heads=2, layers=1, attention_mesh_depth=20, ffn_mesh_depth=17,
         embedding=1),
    dict(vocab_size=9, context=3, width=256, heads=4, layers=1, attention_mesh_depth=18, ffn_mesh_depth=40,
         embedding=1, connectivity=1),
]


@pytest.mark.parametrize("cfg", DEEP, ids=[_ids(c) for c in DEEP])
def test_deep_stacks_match_the_oracle(cfg):
    """At the seeded initialisation a deep stack's gradient all but vanishes, so
    the weights are drawn from U(-1.3, 1.3) instead: every layer carries a
    gradient of order 1e-3..1."""
    g, o = configs_for(**cfg)
    params = np.random.default_rng(3).uniform(-1.3, 1.3, O.parameter_count(o)).astype(np.float32)
    x, y, _ = batch(cfg["vocab_size"], 2, 3)
    ref_loss, ref_grad = O.loss_and_gradient(o, params, x, y, 3)
    assert np.median(np.abs(ref_grad)) > 1e-4
    with G.MeshGpt(0, g, 7) as model:
        model.set_parameters(params)
        loss, grad = model.loss_and_gradient(x, y, 3)
        assert abs(loss - ref_loss) <= TOL * (1 + abs(ref_loss)), (loss, ref_loss)
        assert_close(grad, ref_grad, what="deep stack gradient")


@pytest.mark.parametrize("setting", [dict(learning_rate=0.002, weight_decay=0.01),
                                     dict(learning_rate=0.001, weight_decay=1.0, beta2=0.98)])
@pytest.mark.parametrize("frozen", [0, 1])
def test_adamw_steps(setting, frozen):
    """mesh-gpt.rs:400-470: three steps; each gradient against the oracle on the
    GPU's weights, each update against f32 AdamW on the GPU's own gradient."""
    cfg = dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2,
               frozen=frozen)
    g, o = configs_for(**cfg)
    x = np.array([0, 1, 3, 2, 4, 1], dtype=np.uint32)
    y = (np.array([IGN, IGN, 2, IGN, IGN, 0]) if setting.get("beta2") else np.array([1, 3, 2, 4, 1, 0])).astype(
        np.uint32)
    opts = G.AdamW(**setting)
    skip = O.lib().og_embedding_parameter_count(__import__("ctypes").byref(o)) if frozen else 0
    with G.MeshGpt(0, g, 7) as model:
        cpu = O.Adam(model.parameters(), **setting)
        for step in range(3):
            before = model.parameters()
            _, expected = O.loss_and_gradient(o, before, x, y, 3)
            _, grad = model.loss_and_gradient(x, y, 3)
            assert_close(grad, expected, what=f"step {step} gradient")
            cpu.value = before.copy()
            want = cpu.step(grad, skip=skip)
            model.train_batch(x, y, 3, opts)
            got = model.parameters()
            # The same f32 update on the same inputs; only sqrt and division
            # rounding may differ.
            np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-9)
            if frozen:
                assert np.array_equal(got[:skip], before[:skip])


def test_nonfinite_step_changes_nothing():
    """A step whose loss is not finite stops before AdamW (gpu.rs:2296-2313):
    train_batch raises MG_NONFINITE with the weights, the moments and the step
    count as they were, so the next (finite) steps update exactly as f32 AdamW
    from step 1 on.  The weights make the loss depend on the batch: block 0's V
    mesh scales channel 0 by 3e38 in each of its two ELU layers, so a token
    whose normalised row has n_0 > 0 overflows to inf there (NaN after XSA,
    NaN loss), while a token with n_0 < 0 saturates at ELU = -1 (finite, with a
    zero gradient through that path).  The failing step is replayed from the
    same captured graph as the good ones."""
    cfg = dict(vocab_size=7, context=3, width=8, heads=2, layers=1, attention_mesh_depth=3, ffn_mesh_depth=2)
    g, _ = configs_for(**cfg)
    W, A = 8, 3
    v_mesh = 2 * W * A * 3  # after the embedding, Q and K meshes (config.rs:367-396)
    setting = dict(learning_rate=0.002, weight_decay=0.01)
    opts = G.AdamW(**setting)
    with G.MeshGpt(0, g, 7) as model:
        params = model.parameters()
        for layer in (0, 1):
            params[v_mesh + layer * 2 * W] = 3e38  # channel 0: self weight
            params[v_mesh + layer * 2 * W + 1] = 0.0  # and no partner
        model.set_parameters(params)
        E = model.token_embeddings()
        up = [t for t in range(7) if E[t, 0] > 1e-3]
        down = [t for t in range(7) if E[t, 0] < -1e-3]
        assert up and len(down) >= 2, E[:, 0]
        bad_x = np.array([down[0], up[0], down[1]], np.uint32)
        good_x = np.array([down[0], down[1], down[0]], np.uint32)
        y = np.array([1, 2, 3], np.uint32)
        cpu = O.Adam(params, **setting)
        for step in range(3):
            before = model.parameters()
            with pytest.raises(G.MeshGptError) as err:
                model.train_batch(bad_x, y, 3, opts)
            assert err.value.status == G.MG_NONFINITE
            assert "finite" in str(err.value)
            assert np.array_equal(model.parameters(), before), f"step {step}: a failed step moved the weights"
            loss, grad = model.loss_and_gradient(good_x, y, 3)
            assert np.isfinite(loss) and np.isfinite(grad).all()
            want = cpu.step(grad).copy()
            model.train_batch(good_x, y, 3, opts)
            np.testing.assert_allclose(model.parameters(), want, rtol=2e-6, atol=1e-9,
                                       err_msg=f"step {step}: the update after a failed step")


@pytest.mark.parametrize("geometry", [{}, dict(normalization=2), dict(preserve_features=2)],
                         ids=["default", "normalised", "protected"])
def test_training_then_inference_uses_the_new_weights(geometry):
    """After train_batch the tables derived from the weights are rebuilt before
    the next inference call: logits equal the oracle's on the trained weights.
    With protected coordinates, the weights that would write them stay zero
    (set_parameters accepts the trained vector: config.rs:476-488)."""
    cfg = dict(vocab_size=26, context=32, width=32, heads=4, layers=2, **geometry)
    g, o = configs_for(**cfg)
    x, y, _ = batch(26, 2, 32)
    with G.MeshGpt(0, g, 7) as model:
        before = model.logits(x, 32)
        for _ in range(5):
            model.train_batch(x, y, 32)
        params = model.parameters()
        after = model.logits(x, 32)
        assert not np.allclose(before, after)
        assert_close(after, O.logits(o, params, x, 32), what="logits after training")
        assert_close(model.token_embeddings(), O.token_embeddings(o, params), what="embeddings after training")
        toks = model.generate_tokens(x[None, :16], 4, 0.0, 7)[0]
        assert np.array_equal(toks, O.generate(o, params, x[:16], 4, 0.0, 7, cached=True))
        model.set_parameters(params)


def test_training_trajectory_follows_the_oracle():
    """Twenty AdamW steps of the grok shape (answer-only targets): the GPU's
    losses track the oracle's (f64 gradients, f32 AdamW) step by step."""
    cfg = dict(vocab_size=99, context=4, width=128, heads=4, layers=2)
    g, o = configs_for(**cfg)
    rng = np.random.default_rng(11)
    a, b = rng.integers(0, 97, 64), rng.integers(0, 97, 64)
    x = np.stack([a, np.full(64, 97), b, np.full(64, 98)], 1).reshape(-1).astype(np.uint32)
    y = np.stack([np.full(64, IGN), np.full(64, IGN), np.full(64, IGN), (a + b) % 97], 1).reshape(-1).astype(np.uint32)
    setting = dict(learning_rate=0.001, weight_decay=1.0, beta2=0.98)
    with G.MeshGpt(0, g, 7) as model:
        cpu = O.Adam(model.parameters(), **setting)
        opts = G.AdamW(**setting)
        for step in range(20):
            ref_loss, ref_grad = O.loss_and_gradient(o, cpu.value, x, y, 4)
            loss = model.train_batch(x, y, 4, opts)
            assert abs(loss - ref_loss) <= 1e-4 * (1 + abs(ref_loss)), (step, loss, ref_loss)
            cpu.step(ref_grad)
        np.testing.assert_allclose(model.parameters(), cpu.value, rtol=0, atol=2e-4)


def test_training_rejections_carry_the_reference_messages():
    g, _ = configs_for(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2,
                       ffn_mesh_depth=2)
    x = np.array([0, 1, 3], dtype=np.uint32)
    with G.MeshGpt(0, g, 7) as model:
        cases = [
            (lambda: model.loss_and_gradient(x, np.full(3, IGN, np.uint32), 3),
             "batch must contain at least one supervised target"),
            (lambda: model.loss_and_gradient(x, np.array([0, 1, 9], np.uint32), 3),
             "target ID is outside the vocabulary"),
            (lambda: model.cross_entropy(np.array([0, 7, 1], np.uint32), x, 3), "token ID is outside the vocabulary"),
            (lambda: model.train_batch(x, x, 3, G.AdamW(learning_rate=0.0)),
             "AdamW requires finite positive learning rate/epsilon, nonnegative decay, and betas in [0, 1)"),
            (lambda: model.train_batch(x, x, 3, G.AdamW(beta2=1.0)),
             "AdamW requires finite positive learning rate/epsilon, nonnegative decay, and betas in [0, 1)"),
        ]
        for call, message in cases:
            with pytest.raises(G.MeshGptError) as err:
                call()
            assert message in str(err.value)
        # A rejected step changes nothing.
        before = model.parameters()
        with pytest.raises(G.MeshGptError):
            model.train_batch(x, x, 3, G.AdamW(epsilon=0.0))
        assert np.array_equal(model.parameters(), before)
    wide, _ = configs_for(vocab_size=7, context=3, width=2048, heads=2, layers=1, attention_mesh_depth=1,
                          ffn_mesh_depth=1)
    with G.MeshGpt(0, wide, 7) as model:
        with pytest.raises(G.MeshGptError) as err:
            model.loss_and_gradient(np.zeros(3, np.uint32), np.zeros(3, np.uint32), 3)
        assert err.value.status == G.MG_UNSUPPORTED


def test_reference_default_training_run():
    """The reference's default `mesh-gpt train` (src/bin/mesh-gpt.rs:173-299):
    demo corpus, 1000 AdamW steps, a report every 100.  Step 0 is the published
    3.38668 / 3.37963 (docs/mesh-gpt.md:264); every report follows the oracle's
    f64-gradient run (tests/golden/demo_training.json, written by
    make_demo_training.py) to 1e-4 through step 300, after which the two f32
    update trajectories drift apart by rounding (at most 2.7e-3 observed, bound
    5e-3); step 1000 is within 1e-2 of the published 1.70316 / 1.91340, itself
    a third such trajectory (the CUDA f32 run), 1.3e-3 / 6.8e-3 from the f64 one."""
    import json
    import os

    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "golden", "mesh-gpt-demo.txt"), encoding="utf-8") as f:
        text = f.read()
    chars = sorted(set(text))
    index = {ch: i for i, ch in enumerate(chars)}
    tokens = np.array([index[ch] for ch in text], dtype=np.uint32)
    with open(os.path.join(here, "golden", "demo_training.json")) as f:
        expected = {r["step"]: r for r in json.load(f)["reports"]}
    ex, ey = O.text_batch(tokens, True, 32, 8, 101)
    x0, y0 = O.text_batch(tokens, False, 32, 8, 7)
    with G.MeshGpt(0, G.GptConfig(vocab_size=26), 7) as model:
        reports = {0: (model.cross_entropy(x0, y0, 32), model.cross_entropy(ex, ey, 32))}
        assert abs(reports[0][0] - 3.38668) <= 1e-5 and abs(reports[0][1] - 3.37963) <= 1e-5
        opts = G.AdamW(learning_rate=0.003, weight_decay=0.01)
        total, count = 0.0, 0
        for step in range(1, 1001):
            x, y = O.text_batch(tokens, False, 32, 8, 7 + step)
            total += model.train_batch(x, y, 32, opts)
            count += 1
            if step % 100 == 0:
                reports[step] = (total / count, model.cross_entropy(ex, ey, 32))
                total, count = 0.0, 0
    for step, (train, valid) in reports.items():
        bound = 1e-4 if step <= 300 else 5e-3
        assert abs(train - expected[step]["train"]) <= bound, (step, train, expected[step])
        assert abs(valid - expected[step]["validation"]) <= bound, (step, valid, expected[step])
    assert abs(reports[1000][0] - 1.70316) <= 1e-2 and abs(reports[1000][1] - 1.91340) <= 1e-2


def test_cli_train_default_run(tmp_path):
    """`mesh-gpt train` with every default (src/bin/mesh-gpt.rs:173-299) on the
    demo corpus: its stdout lines, loss.csv, geometry.txt, run.txt, checkpoint
    and sample.txt.  The reports are those of the same loop run through the
    library (the golden trajectory and the published step 0 / 1000, as in
    test_reference_default_training_run), and the checkpoint holds exactly the
    weights that loop produces."""
    import json
    import os
    import re
    import subprocess

    here = os.path.dirname(os.path.abspath(__file__))
    corpus = os.path.join(here, "golden", "mesh-gpt-demo.txt")
    out = tmp_path / "run"
    res = subprocess.run([G.CLI_PATH, "train", "--dataset", corpus, "--output", str(out)], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    head, sep, rest = res.stdout.partition(f"Saved checkpoint to {out / 'model.bin'}\n\n")
    assert sep and rest.endswith("\n")
    lines = head.splitlines()
    assert lines[0] == "Mesh GPT: blocks=2, width=32, heads=4, context=32, vocabulary=26, parameters=3072"
    assert lines[1] == ("Meshes: Q/K/V/output depth=4, FFN depth=6; embeddings=mesh, form=parity, norm=none, "
                        "protected=0; RoPE=true, QK-Norm=true, XSA=true")
    pattern = re.compile(r"step +(\d+): train CE=(\d+\.\d{5}), validation CE=(\d+\.\d{5}), perplexity=(\d+\.\d{3})$")
    reports = {}
    for line in lines[2:13]:
        m = pattern.match(line)
        assert m and len(line.split(":")[0]) == len("step ") + 6, line
        reports[int(m.group(1))] = tuple(float(v) for v in m.groups()[1:])
    assert sorted(reports) == list(range(0, 1001, 100))
    assert re.fullmatch(r"Training time: \d+\.\d{3} s", lines[13]) and len(lines) == 14
    with open(os.path.join(here, "golden", "demo_training.json")) as f:
        expected = {r["step"]: r for r in json.load(f)["reports"]}
    for step, (train, valid, ppl) in reports.items():
        bound = 1e-4 if step <= 300 else 5e-3
        assert abs(train - expected[step]["train"]) <= bound + 5e-6, (step, train)
        assert abs(valid - expected[step]["validation"]) <= bound + 5e-6, (step, valid)
        assert abs(ppl - np.exp(valid)) <= 2e-4 * ppl
    # docs/mesh-gpt.md:264-266
    assert abs(reports[0][0] - 3.38668) <= 1e-5 and abs(reports[0][1] - 3.37963) <= 1e-5
    assert abs(reports[1000][0] - 1.70316) <= 1e-2 and abs(reports[1000][1] - 1.91340) <= 1e-2

    rows = (out / "loss.csv").read_text().splitlines()
    assert rows[0] == "step,train_cross_entropy,validation_cross_entropy,validation_perplexity"
    csv = {int(r.split(",")[0]): [float(v) for v in r.split(",")[1:]] for r in rows[1:]}
    assert sorted(csv) == sorted(reports)
    for step, (train, valid, ppl) in csv.items():
        assert abs(train - reports[step][0]) <= 5e-6 and abs(valid - reports[step][1]) <= 5e-6
        assert abs(ppl - np.exp(valid)) <= 1e-8 * ppl

    assert (out / "geometry.txt").read_text() == (
        "embedding_form=parity\nembedding_order=token\nembedding_frequency=1\nembedding_harmonics=1\n"
        "equiangular_overlap=0\nembedding_norm=none\nfreeze_embedding=false\npreserve_features=0\n"
        "geometry_modulus=0\ngeometry_seed=0\nrope=true\nqk_norm_enabled=true\nxsa_enabled=true\n"
        "geometry_supplies_arithmetic_order=false\n")
    run = dict(line.split("=", 1) for line in (out / "run.txt").read_text().splitlines())
    fixed = dict(attention="xsa", positions="slice_rope", rope_base="10000", normalization="pre_rmsnorm",
                 rmsnorm_epsilon="1e-5", rmsnorm_affine="false", qk_norm="per_head_rmsnorm", bias="false",
                 embeddings="mesh", token_codes="signed_binary_parity_radix",
                 embedding_depth="attention_mesh_depth", head="tied_mesh_embeddings", all_parameters="mesh_edges",
                 dataset=corpus, seed="7", steps="1000", batch="8", width="32", heads="4", layers="2", context="32",
                 attention_mesh_depth="4", ffn_mesh_depth="6", parameters="3072", learning_rate="0.003",
                 weight_decay="0.01")
    for key, value in fixed.items():
        assert run.pop(key) == value, key
    assert abs(float(run.pop("initial_validation_cross_entropy")) - csv[0][1]) <= 1e-9
    assert abs(float(run.pop("final_validation_cross_entropy")) - csv[1000][1]) <= 1e-9
    assert float(run.pop("training_seconds")) > 0 and not run

    # The same loop through the library: batches from the product's TextDataset
    # (checked against the oracle's on the CPU), seeds 7 + step.
    saved = G.Checkpoint.load(str(out / "model.bin"))
    cfg = G.GptConfig(vocab_size=26)
    assert saved.config == cfg
    text = open(corpus, encoding="utf-8").read()
    tokenizer = G.CharacterTokenizer.from_text(text)
    assert G.CharacterTokenizer(saved.characters) == tokenizer
    tokens = np.array(tokenizer.encode(text), dtype=np.uint32)
    with G.MeshGpt(0, cfg, 7) as model:
        for step in range(1, 1001):
            x, y = G.text_batch(tokens, cfg, False, 32, 8, 7 + step)
            model.train_batch(x, y, 32)
        assert np.array_equal(model.parameters().view(np.uint32), saved.parameters.view(np.uint32))
        sample = model.generate(tokenizer.characters, "the little robot ", 240, 0.7, 7)
    assert (out / "sample.txt").read_text(encoding="utf-8") == sample == rest[:-1]


def test_bench_binary_reference_protocol(tmp_path):
    """mesh-gpt-bench with the reference's documented command
    (docs/cuda-performance.md:25-28, two trials here): each trial restores the
    seeded weights, so both print the same losses, and those are the losses of
    the same protocol run through the library (bench.py's training figure);
    timings.csv, run.txt and the first trial's model.bin hold what they should,
    the checkpoint with the equation dataset's tokenizer (grokking.rs:146-157)."""
    import os
    import re
    import subprocess

    bench = os.path.join(os.path.dirname(G.CLI_PATH), "mesh-gpt-bench")
    out = tmp_path / "bench"
    res = subprocess.run([bench, "--steps", "30", "--warmup", "10", "--trials", "2", "--output", str(out)],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.splitlines()
    pat = re.compile(r"trial (\d): (\d+\.\d{3}) ms/update; (\d+) tokens/s; CE (\d+\.\d{5}) -> (\d+\.\d{5})$")
    m1, m2 = pat.match(lines[0]), pat.match(lines[2])
    assert m1 and m2 and re.fullmatch(r"device buffers: \d+\.\d MiB", lines[1]) and len(lines) == 3, lines
    assert m1.group(4, 5) == m2.group(4, 5)

    cfg = G.GptConfig(vocab_size=99, context=4, width=128, heads=4, layers=2)
    n_train, _ = G.equation_split()
    x, y = G.equation_batch(np.arange(512) % n_train)
    opts = G.AdamW(learning_rate=0.001, weight_decay=1.0, beta2=0.98)
    with G.MeshGpt(0, cfg, 7) as model:
        for _ in range(10):
            model.train_batch(x, y, 4, opts)
        losses = [model.train_batch(x, y, 4, opts) for _ in range(30)]
        params = model.parameters()
    assert m1.group(4) == f"{losses[0]:.5f}" and m1.group(5) == f"{losses[-1]:.5f}"

    rows = (out / "timings.csv").read_text().splitlines()
    assert rows[0] == "trial,steps,total_ms,ms_per_step,first_loss,last_loss,weight_l2" and len(rows) == 3
    t1 = rows[1].split(",")
    assert t1[:2] == ["1", "30"] and abs(float(t1[4]) - losses[0]) <= 1e-9 and abs(float(t1[5]) - losses[-1]) <= 1e-9
    assert abs(float(t1[6]) - np.sqrt(np.sum(params.astype(np.float64) ** 2))) <= 1e-6
    run = dict(line.split("=", 1) for line in (out / "run.txt").read_text().splitlines())
    for key, value in dict(precision="fp32", workload="add_mod97", seed="7", width="128", heads="4", layers="2",
                           attention_mesh_depth="4", ffn_mesh_depth="6", vocabulary="99", context="4", batch="512",
                           steps="30", warmup="10", trials="2", learning_rate="0.001", weight_decay="1",
                           betas="0.9,0.98", timing="end_to_end_wall_clock",
                           final_parameter_download="included").items():
        assert run[key] == value, key
    assert int(run["allocated_device_bytes"]) > 0

    saved = G.Checkpoint.load(str(out / "model.bin"))
    assert saved.config == cfg
    assert np.array_equal(saved.parameters.view(np.uint32), params.view(np.uint32))
    perm, _, _ = __import__("test_host_train").oracle_equations(97, 0, 0.5, 7)
    want = [" "] * 99
    for residue, token in enumerate(perm):
        want[token] = chr(0xE000 + residue)
    want[97], want[98] = "+", "="
    assert G.CharacterTokenizer(saved.characters) == G.CharacterTokenizer(want)

    # Other contexts take the cyclic next-token workload (mesh-gpt-bench.rs:140-149).
    res = subprocess.run([bench, "--context", "8", "--batch", "16", "--steps", "2", "--warmup", "1", "--trials", "1",
                          "--output", str(tmp_path / "cyclic")], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert "workload=cyclic_next_token" in (tmp_path / "cyclic" / "run.txt").read_text()


def test_cli_grok_published_epoch(tmp_path):
    """The documented one-epoch grok run (docs/grokking.md:12-14, 190-195):
    4704 training equations in nine batches of 512 and one of 96, warmup over
    the 10 updates, both complete splits evaluated at steps 0 and 10.  The
    reference's CUDA run printed train CE 7.41967 -> 6.53287 and validation
    CE 7.43258 -> 6.54729 with answer accuracy zero; step 0 is also the
    published full-split 7.419670094 / 7.432581042 (docs/cuda-performance.md:238-240).
    Artifacts as listed in docs/grokking.md:139-166."""
    import os
    import re
    import subprocess

    out = tmp_path / "grok"
    res = subprocess.run([G.CLI_PATH, "grok", "--epochs", "1", "--report-every", "10", "--output", str(out)],
                         capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.splitlines()
    assert lines[0] == "Mesh GPT grokking: add mod 97, train=4704, validation=4705, batch=512, parameters=12288"
    assert lines[1] == "Answer-only loss; AdamW beta2=0.98, decay=1, warmup=10; continuing for 10 updates"
    pat = re.compile(r"step +(\d+): train CE=(\d+\.\d{5}) accuracy=(\d+\.\d\d)%; "
                     r"validation CE=(\d+\.\d{5}) accuracy=(\d+\.\d\d)%$")
    m0, m10 = pat.match(lines[2]), pat.match(lines[3])
    assert m0 and m10 and m0.group(1) == "0" and m10.group(1) == "10", lines
    assert len(lines[2].split(":")[0]) == len("step ") + 7
    assert lines[4:] == [f"Saved model, split, symbols, embeddings, predictions, and learning curves to {out}",
                         "First recorded accuracy >=99%: train=not_reached, validation=not_reached",
                         "Stopped after 10 updates: update_budget"]
    rows = (out / "loss.csv").read_text().splitlines()
    assert rows[0] == ("step,training_examples_seen,completed_epochs,examples_in_partial_epoch,train_cross_entropy,"
                       "validation_cross_entropy,train_accuracy,validation_accuracy,weight_l2,learning_rate,"
                       "elapsed_seconds")
    r0, r10 = (r.split(",") for r in rows[1:])
    assert r0[:4] == ["0", "0", "0", "0"] and r10[:4] == ["10", "4704", "1", "0"]
    assert abs(float(r0[4]) - 7.419670094) <= 1e-5 and abs(float(r0[5]) - 7.432581042) <= 1e-5
    assert abs(float(r10[4]) - 6.53287) <= 5e-6 and abs(float(r10[5]) - 6.54729) <= 5e-6
    assert float(r10[7]) == 0.0 and r10[9] == "0.001000000" and r0[9] == "0.000000000"
    assert m10.group(5) == "0.00"
    run = dict(line.split("=", 1) for line in (out / "run.txt").read_text().splitlines())
    for key, value in dict(status="complete", operation="add", modulus="97", train_fraction="0.5",
                           training_equations="4704", validation_equations="4705", seed="7", width="128",
                           parameters="12288", embedding_parameters="1024", all_parameters="mesh_edges",
                           attention="xsa", positions="slice_rope", qk_norm="per_head_rmsnorm", embeddings="mesh",
                           mesh_connectivity="neighbor", learning_rate="0.001", weight_decay="1", batch="512",
                           steps="10", report_every="10", requested_epochs="1", steps_per_epoch="10",
                           stop_validation_accuracy="none", evaluation_batch="128", initialization_gain="1",
                           embedding_output_gain="1", embedding_init_unit="false", qk_signs="0",
                           workspace_capacity="1", stop_reason="update_budget", completed_steps="10",
                           training_examples_seen="4704", completed_epochs="1", examples_in_partial_epoch="0",
                           first_recorded_train_99_step="not_reached",
                           first_recorded_validation_99_step="not_reached", embedding_form="parity",
                           xsa_enabled="true").items():
        assert run[key] == value, key
    eq = (out / "equations.csv").read_text().splitlines()
    assert eq[0] == "split,pair_id,a,b,answer,input_a_id,operator_id,input_b_id,equals_id,target_id"
    assert len(eq) == 1 + 9409 and sum(r.startswith("train,") for r in eq) == 4704
    perm, _, _ = __import__("test_host_train").oracle_equations(97, 0, 0.5, 7)
    for r in eq[1:50]:
        split, pair, a, b, ans, ia, op, ib, eqs, tgt = r.split(",")
        assert int(pair) == 97 * int(a) + int(b) and int(ans) == (int(a) + int(b)) % 97
        assert (int(ia), int(op), int(ib), int(eqs), int(tgt)) == (perm[int(a)], 97, perm[int(b)], 98, perm[int(ans)])
    sym = (out / "symbols.csv").read_text().splitlines()
    assert sym[0] == "token_id,symbol" and sym[98] == "97,add" and sym[99] == "98,="
    assert sym[1 + int(perm[5])] == f"{perm[5]},5"
    pred = (out / "predictions.csv").read_text().splitlines()
    assert pred[0] == "split,a,b,answer,prediction,correct,cross_entropy" and len(pred) == 1 + 9409
    emb = (out / "embeddings.csv").read_text().splitlines()
    assert len(emb) == 100 and emb[0].startswith("token_id,symbol,c0,c1") and emb[0].endswith(",c127")
    initial = G.Checkpoint.load(str(out / "initial-model.bin"))
    final = G.Checkpoint.load(str(out / "model.bin"))
    o = O.config(vocab_size=99, context=4, width=128, heads=4, layers=2)
    assert np.array_equal(initial.parameters.view(np.uint32), O.initialize(o, 7).view(np.uint32))
    assert not np.array_equal(final.parameters, initial.parameters)
    # The final embeddings are those of the saved weights.
    with G.MeshGpt(0, final.config, 7) as model:
        model.set_parameters(final.parameters)
        vectors = model.token_embeddings()
    row5 = [float(v) for v in emb[1 + int(perm[5])].split(",")[2:]]
    np.testing.assert_allclose(row5, vectors[int(perm[5])], rtol=0, atol=1e-9)


def test_cli_grok_published_1000_updates(tmp_path):
    """The documented 1000-update smoke run of the default grok model
    (docs/grokking.md:197-200): the reference's CUDA run ended at training
    cross-entropy 4.58679 / accuracy 1.28% and validation 4.59957 / 0.83%,
    which this run prints to every digit (1000 f32 AdamW updates of 512
    equations, warmup, seeded epoch shuffles)."""
    import subprocess

    res = subprocess.run([G.CLI_PATH, "grok", "--steps", "1000", "--output", str(tmp_path / "grok")],
                         capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.splitlines()
    assert lines[2] == "step       0: train CE=7.41967 accuracy=0.00%; validation CE=7.43258 accuracy=0.00%"
    assert lines[3] == "step    1000: train CE=4.58679 accuracy=1.28%; validation CE=4.59957 accuracy=0.83%"
    assert lines[-1] == "Stopped after 1000 updates: update_budget"


def test_cli_grok_initialisation_controls(tmp_path):
    """grok's initialisation controls (src/bin/mesh-gpt/grokking.rs:221-283),
    all at once: every mesh edge scaled by --init-gain, the embedding mesh's
    final layer by --embedding-output-gain, the final Q and K mesh rows by
    seeded signs (their own SplitMix64 stream), the table taken from the
    adjusted mesh's vectors, and each table row normalised once.  The
    step-zero checkpoint holds exactly that, restated here from the oracle's
    seeded initialisation and token vectors."""
    import subprocess

    out = tmp_path / "grok"
    res = subprocess.run([G.CLI_PATH, "grok", "--steps", "1", "--report-every", "1", "--init-gain", "1.5",
                          "--embedding-output-gain", "0.5", "--qk-signs", "1", "--embedding", "table",
                          "--embedding-init-unit", "--output", str(out)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    W, A, F, L, V = 128, 4, 6, 2, 99
    mesh = O.config(vocab_size=V, context=4, width=W, heads=4, layers=L)
    p = O.initialize(mesh, 7) * np.float32(1.5)
    emb = 2 * W * A
    p[emb - 2 * W:emb] *= np.float32(0.5)
    mask = (1 << 64) - 1
    state = 7 ^ 0x514B5349474E5331
    block = 2 * W * (4 * A + F)
    for b in range(L):
        for proj in range(2):
            end = emb + b * block + (proj + 1) * emb
            for i in range(end - 2 * W, end, 2):
                state = (state + 0x9E3779B97F4A7C15) & mask
                z = state
                z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
                z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
                z ^= z >> 31
                if z >> 63:
                    p[i] = -p[i]
                    p[i + 1] = -p[i + 1]
    table = O.token_embeddings(mesh, p)
    table = (table / np.sqrt(np.sum(table ** 2, axis=1, keepdims=True))).astype(np.float32)
    saved = G.Checkpoint.load(str(out / "initial-model.bin"))
    assert saved.parameters.size == V * W + p.size - emb
    np.testing.assert_allclose(saved.parameters[:V * W].reshape(V, W), table, rtol=0, atol=2e-7)
    assert np.array_equal(saved.parameters[V * W:].view(np.uint32), p[emb:].view(np.uint32))
    run = dict(line.split("=", 1) for line in (out / "run.txt").read_text().splitlines())
    assert (run["initialization_gain"], run["embedding_output_gain"], run["qk_signs"], run["embedding_init_unit"],
            run["embeddings"], run["all_parameters"]) == ("1.5", "0.5", "1", "true", "table",
                                                            "mesh_edges_and_token_table")


def test_cli_grok_stop_rule_and_epoch_tails(tmp_path):
    """--stop-validation-accuracy ends at the first report whose complete
    validation split reaches the target, else the budget runs out
    (grokking.rs:386-422); examples seen count short epoch tails
    (mod 5 at fraction 0.8: 20 training equations, batches of 6, so epochs
    of 6 + 6 + 6 + 2)."""
    import subprocess

    out = tmp_path / "grok"
    res = subprocess.run([G.CLI_PATH, "grok", "--modulus", "5", "--train-fraction", "0.8", "--batch", "6",
                          "--steps", "400", "--report-every", "4", "--stop-validation-accuracy", "0.4",
                          "--output", str(out)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    rows = [r.split(",") for r in (out / "loss.csv").read_text().splitlines()[1:]]
    steps = [int(r[0]) for r in rows]
    assert steps == list(range(0, 4 * len(rows), 4))
    for r in rows:  # four updates per epoch of 20 equations
        step, seen = int(r[0]), int(r[1])
        assert seen == 20 * (step // 4) and int(r[2]) == step // 4 and int(r[3]) == 0
    reached = [i for i, r in enumerate(rows) if float(r[7]) >= 0.4]
    run = dict(line.split("=", 1) for line in (out / "run.txt").read_text().splitlines())
    if reached:
        assert reached[0] == len(rows) - 1 and run["stop_reason"] == "validation_accuracy"
        assert res.stdout.splitlines()[-1] == f"Stopped after {steps[-1]} updates: validation_accuracy"
    else:
        assert steps[-1] == 400 and run["stop_reason"] == "update_budget"
    assert run["completed_steps"] == str(steps[-1]) and run["steps_per_epoch"] == "4"
