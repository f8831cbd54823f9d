"""`mesh-gpt verify` for this build: the GPU path against the CPU oracle.

The reference's `verify` command (src/bin/mesh-gpt.rs:624-896) checks its
CUDA path against its f64 CPU reference on a fixed list of models and prints
one PASS line per model.  The product CLI of this build does not link the
oracle (test infrastructure only), so the command lives here, beside the
tests, and drives the product through its C ABI (grokking_abmod_amd):

- verify_model (mesh-gpt.rs:324-553) on the reference's model list
  (mesh-gpt.rs:651-857) and its geometry list (every embedding form with mesh
  and table embeddings, overlap 0.25, mesh-gpt.rs:898-960): effective
  embeddings, logits of x[i] = i % V for each (batch, sequence) case, loss and
  every gradient for targets (i + 2) % V and answer-only, causality and prefix
  invariance, the rejected inputs, three AdamW steps under each of the two
  optimizer settings (against f32 AdamW on the GPU's own gradient) and a reset,
  and the zero-embedding behaviour (or, with protected coordinates, the codes
  that survive zero weights);
- every value within TOL * (1 + |ref|), TOL = 1e-4 (the reference uses 5e-4).

Not repeated here: the reference's isolated-kernel and workspace-cache checks
(mesh-gpt.rs:555-622 and gpu.rs's verify_* functions), which test kernels and
buffers of its CUDA launcher that this build does not have; tests/ holds the
corresponding checks of this build's kernels.

Usage: python tests/verify.py [--device N] [--quick]
Exit status 0 when every model passes, 1 at the first failure (its message on
stderr, as the reference's Err).
"""
import argparse
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))

import grokking_abmod_amd as G  # noqa: E402
import oracle_lib as O  # noqa: E402

TOL = 1e-4
IGN = G.IGNORE_TARGET
FORMS = ["parity", "circle", "fourier", "orthogonal", "simplex", "equiangular", "antipodal", "hypercube",
         "signed-permutations", "sphere"]


class Failure(Exception):
    pass


def close(name, expected, actual, tolerance=TOL):
    """mesh-gpt.rs:314-322 over arrays: finite and |e - a| <= tol (1 + |e|)."""
    e = np.asarray(expected, dtype=np.float64)
    a = np.asarray(actual, dtype=np.float64)
    bad = ~(np.isfinite(e) & np.isfinite(a) & (np.abs(e - a) <= tolerance * (1.0 + np.abs(e))))
    if bad.any():
        i = np.unravel_index(int(np.argmax(bad)), bad.shape)
        raise Failure(f"{name} {i}: expected {e[i]:.9f}, got {a[i]:.9f}")


def model_list():
    from test_gpu_parity import VERIFY  # the reference's list, mesh-gpt.rs:651-857

    models = [(cfg, cases) for cfg, cases in VERIFY]
    base = dict(vocab_size=7, context=5, width=8, heads=2, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2)
    for form in range(len(FORMS)):
        for embedding in (0, 1):
            models.append((dict(base, form=form, overlap=0.25, embedding=embedding), [(1, 1), (2, 3), (3, 5)]))
    return models


def verify_model(device, cfg, cases):
    g, o = G.GptConfig(**cfg), O.config(**cfg)
    params = O.initialize(o, 7)
    V = cfg["vocab_size"]
    with G.MeshGpt(device, g, 7) as model:
        if not np.array_equal(model.parameters(), params):
            raise Failure("seeded parameters differ from the reference initialisation")
        close("effective embedding", O.token_embeddings(o, params), model.token_embeddings())
        for batch, sequence in cases:
            x = (np.arange(batch * sequence) % V).astype(np.uint32)
            y = ((np.arange(batch * sequence) + 2) % V).astype(np.uint32)
            close(f"logits b={batch} s={sequence}", O.logits(o, params, x, sequence), model.logits(x, sequence))
            if g.preserve_features > 0:
                codes = O.token_codes(o)
                states = model.hidden_states(x, sequence)
                k = g.preserve_features
                if not np.array_equal(states[:, :k], codes[x][:, :k]):
                    raise Failure("protected feature changed inside the residual stack")
            answer = np.where(np.arange(x.size) % sequence == sequence - 1, y, IGN).astype(np.uint32)
            for targets in (y, answer):
                ref_loss, ref_grad = O.loss_and_gradient(o, params, x, targets, sequence)
                loss, grad = model.loss_and_gradient(x, targets, sequence)
                close("cross-entropy", ref_loss, loss)
                close("gradient", ref_grad, grad)
        if V >= 5:
            full = model.logits([0, 1, 2], 3)
            changed = model.logits([0, 1, 4], 3)
            if not (np.array_equal(full[:2], changed[:2]) and np.array_equal(full[:2], model.logits([0, 1], 2))):
                raise Failure("causal mask leaked future tokens")
        for call in (lambda: model.logits([], 1), lambda: model.logits([2**32 - 1], 1),
                     lambda: model.logits([0], 0),
                     lambda: model.loss_and_gradient([0], [2**32 - 1], 1),
                     lambda: model.set_parameters([0.0])):
            try:
                call()
            except G.MeshGptError:
                continue
            raise Failure("GPT validation failed")
        if V >= 5 and cfg.get("context", 32) >= 3:
            x = np.array([0, 1, 3, 2, 4, 1], dtype=np.uint32)
            skip = O.lib().og_embedding_parameter_count(ctypes.byref(o)) if g.frozen else 0
            for setting in (dict(learning_rate=0.002, weight_decay=0.01),
                            dict(learning_rate=0.001, weight_decay=1.0, beta2=0.98)):
                y = np.array([IGN, IGN, 2, IGN, IGN, 0] if "beta2" in setting else [1, 3, 2, 4, 1, 0], np.uint32)
                model.set_parameters(params)
                cpu = O.Adam(params, **setting)
                first = None
                for step in range(3):
                    _, grad = model.loss_and_gradient(x, y, 3)
                    want = cpu.step(grad, skip=skip).copy()
                    model.train_batch(x, y, 3, G.AdamW(**setting))
                    got = model.parameters()
                    close(f"AdamW step={step}", want, got, 2e-6)
                    if step == 0:
                        first = got
                model.set_parameters(params)
                model.train_batch(x, y, 3, G.AdamW(**setting))
                if not np.array_equal(model.parameters(), first):
                    raise Failure("AdamW reset")
            if g.preserve_features == 0:
                zero = np.full(O.parameter_count(o), 0.5, dtype=np.float32)
                zero[:O.lib().og_embedding_parameter_count(ctypes.byref(o))] = 0.0
                model.set_parameters(zero)
                if np.any(model.logits(x, 3) != 0.0):
                    raise Failure("zero token embeddings produced additive logit offsets")
            else:
                # The fixed injected code survives even if every learned weight is zero.
                model.set_parameters(np.zeros(O.parameter_count(o), dtype=np.float32))
                k = g.preserve_features
                if not np.array_equal(model.hidden_states(x, 3)[:, :k], O.token_codes(o)[x][:, :k]):
                    raise Failure("protected code disappeared with zero learned weights")
    emb = "table" if cfg.get("embedding", 0) else "mesh"
    conn = "butterfly" if cfg.get("connectivity", 0) else "neighbor"
    flag = lambda k: str(bool(cfg.get(k, 1))).lower()  # noqa: E731
    print(f"PASS {emb} embeddings, {conn} meshes, form={FORMS[cfg.get('form', 0)]} "
          f"norm={['none', 'unit', 'rms'][cfg.get('normalization', 0)]} protected={cfg.get('preserve_features', 0)} "
          f"frozen={str(bool(cfg.get('frozen', 0))).lower()} RoPE={flag('rope')} QK={flag('qk_norm')} "
          f"XSA={flag('xsa')} width={cfg['width']} heads={cfg['heads']} layers={cfg['layers']}: logits, "
          "dense/masked gradients, causality, batch tails, AdamW beta2=0.999/0.98/reset, zero-weight behavior",
          flush=True)


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--device", type=int, default=0)
    parser.add_argument("--quick", action="store_true", help="the first three models and one geometry")
    args = parser.parse_args(argv)
    models = model_list()
    if args.quick:
        models = models[:3] + models[-1:]
    try:
        for cfg, cases in models:
            verify_model(args.device, cfg, cases)
    except (Failure, G.MeshGptError) as e:
        print(f'Error: "{e}"', file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
