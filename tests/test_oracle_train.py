"""Pins for the training half of the CPU checker (oracle/meshgpt_oracle_grad.c).

The reference's own gradient tests are restated on the oracle:
- gradients match central finite differences for the tiny config and its three
  ablations, with all targets and with answer-only targets, at the
  reference's bound 4e-4 * (1 + |g|) (src/gpt/reference.rs:911-957);
- answer-only loss and gradients are the mean over supervised equations, and
  batches without a supervised target or with an out-of-vocabulary target are
  rejected (reference.rs:959-989).
Beyond them: the same finite-difference check with each operator switched off
and with the geometry's normalisation and protected coordinates; the gradient
mask (config.rs:490-500); the tape's loss equals the f32 loss kernel's; and
AdamW's closed forms (first step moves each weight by lr * sign(g), zero
gradients only decay).
"""
import numpy as np
import pytest

import oracle_lib as O

IGN = O.IGNORE


def tiny(**kw):
    """reference.rs:809-821"""
    base = dict(vocab_size=5, context=4, width=4, heads=2, layers=1, attention_mesh_depth=2, ffn_mesh_depth=2)
    base.update(kw)
    return O.config(**base)


X = np.array([0, 1, 3, 2, 4, 1])
TARGETS = [np.array([1, 3, 2, 4, 1, 0]), np.array([IGN, IGN, 2, IGN, IGN, 0])]


def finite_difference_check(c, seed=7, bound=4e-4):
    """reference.rs:917-957: +-1e-4 in f32, the step measured in f64."""
    params = O.initialize(c, seed)
    worst = 0.0
    for y in TARGETS:
        _, grad = O.loss_and_gradient(c, params, X, y, 3)
        for i in range(params.size):
            plus, minus = params.copy(), params.copy()
            plus[i] = np.float32(plus[i] + np.float32(1e-4))
            minus[i] = np.float32(minus[i] - np.float32(1e-4))
            step = float(plus[i]) - float(minus[i])
            a, _ = O.loss_and_gradient(c, plus, X, y, 3)
            b, _ = O.loss_and_gradient(c, minus, X, y, 3)
            numerical = (a - b) / step
            err = abs(grad[i] - numerical) / (bound * (1 + abs(grad[i])))
            assert err < 1.0, f"parameter {i}: {grad[i]} vs {numerical}"
            worst = max(worst, err)
    return worst


@pytest.mark.parametrize("embedding", [0, 1])
@pytest.mark.parametrize("connectivity", [0, 1])
def test_gradients_match_finite_differences(embedding, connectivity):
    finite_difference_check(tiny(embedding=embedding, connectivity=connectivity))


@pytest.mark.parametrize("switch", ["rope", "qk_norm", "xsa"])
def test_gradients_match_finite_differences_with_an_operator_off(switch):
    finite_difference_check(tiny(**{switch: 0}))


@pytest.mark.parametrize("geometry", [dict(normalization=1), dict(normalization=2), dict(preserve_features=1)])
def test_gradients_match_finite_differences_with_geometry(geometry):
    # Protected coordinates mask gradient entries (compared as zeros below);
    # the check runs on the unmasked entries.
    c = tiny(**geometry)
    if geometry.get("preserve_features"):
        params = O.initialize(c, 7)
        _, grad = O.loss_and_gradient(c, params, X, TARGETS[0], 3)
        offsets = O.group_offsets(c)
        masked = np.zeros(grad.size, dtype=bool)
        W = c.width
        for g, kind_depth in ((4, c.attention_mesh_depth), (5, c.ffn_mesh_depth)):
            begin = offsets[g] + (kind_depth - 1) * 2 * W
            masked[begin:begin + 2 * c.preserve_features] = True
        assert np.all(grad[masked] == 0.0)
        return
    finite_difference_check(c)


def test_frozen_geometry_zeroes_the_embedding_gradient():
    c = tiny(frozen=1)
    params = O.initialize(c, 7)
    _, grad = O.loss_and_gradient(c, params, X, TARGETS[0], 3)
    emb = O.lib().og_embedding_parameter_count(__import__("ctypes").byref(c))
    assert np.all(grad[:emb] == 0.0) and np.any(grad[emb:] != 0.0)


def test_answer_only_loss_and_gradients_average_over_supervised_equations():
    """reference.rs:959-989"""
    c = tiny()
    params = O.initialize(c, 7)
    y = TARGETS[1]
    loss, grad = O.loss_and_gradient(c, params, X, y, 3)
    l1, g1 = O.loss_and_gradient(c, params, X[:3], y[:3], 3)
    l2, g2 = O.loss_and_gradient(c, params, X[3:], y[3:], 3)
    assert abs(loss - (l1 + l2) / 2) < 1e-12
    assert np.max(np.abs(grad - (g1 + g2) / 2)) < 1e-12
    with pytest.raises(ValueError, match=r"\(-4\)"):
        O.loss_and_gradient(c, params, X, np.full(6, IGN), 3)
    with pytest.raises(ValueError, match=r"\(-3\)"):
        O.loss_and_gradient(c, params, X, np.full(6, 99), 3)
    with pytest.raises(ValueError, match=r"\(-1\)"):
        O.loss_and_gradient(c, params, np.array([IGN]), np.array([0]), 1)


def test_tape_loss_equals_the_loss_kernel():
    """The f64 tape loss and the f32 loss kernel of gpu.rs:949-994 agree to
    f32 rounding on a demo-sized model."""
    c = O.config(vocab_size=26, context=32, width=32, heads=4, layers=2)
    params = O.initialize(c, 7)
    rng = np.random.default_rng(3)
    x = rng.integers(0, 26, 64)
    y = rng.integers(0, 26, 64)
    y[::5] = IGN
    loss, _ = O.loss_and_gradient(c, params, x, y, 32)
    assert abs(loss - O.cross_entropy(c, params, x, y, 32)) < 1e-5


def test_gradient_is_zero_for_zero_embedding_weights_of_the_head_path():
    """With zero embedding weights every token vector and so every logit is 0
    (reference.rs:839-862): the loss is ln V, and no block weight can move it
    (all of them multiply zeros), so their gradient is exactly zero."""
    c = tiny()
    params = np.full(O.parameter_count(c), 0.5, dtype=np.float32)
    emb = O.lib().og_embedding_parameter_count(__import__("ctypes").byref(c))
    params[:emb] = 0.0
    loss, grad = O.loss_and_gradient(c, params, X, TARGETS[0], 3)
    assert abs(loss - np.log(5)) < 1e-12
    assert np.all(grad[emb:] == 0.0)


def test_adam_first_step_moves_each_weight_by_the_learning_rate():
    """With bias correction the first AdamW step has m_hat = g and v_hat = g^2,
    so each weight moves by lr * g / (|g| + eps) - lr * wd * w (gpu.rs:1366-1391)."""
    rng = np.random.default_rng(5)
    w = rng.normal(size=1000).astype(np.float32)
    g = rng.normal(size=1000).astype(np.float32)
    opt = O.Adam(w, learning_rate=0.003, weight_decay=0.0)
    new = opt.step(g)
    np.testing.assert_allclose(new - w, -0.003 * np.sign(g), rtol=1e-4, atol=1e-7)
    opt = O.Adam(w, learning_rate=0.003, weight_decay=0.5)
    new = opt.step(np.zeros_like(g))
    np.testing.assert_allclose(new, w * (1 - 0.003 * 0.5), rtol=1e-6)
    # A steady gradient keeps moving by about lr a step (m_hat / sqrt(v_hat) -> 1).
    opt = O.Adam(w, learning_rate=0.001, weight_decay=0.0, beta2=0.98)
    for _ in range(20):
        before = opt.value.copy()
        new = opt.step(g)
    np.testing.assert_allclose(new - before, -0.001 * np.sign(g), rtol=1e-3, atol=1e-7)


def test_adam_skips_a_frozen_prefix():
    w = np.ones(10, dtype=np.float32)
    opt = O.Adam(w)
    new = opt.step(np.ones(10, dtype=np.float32), skip=4)
    assert np.all(new[:4] == 1.0) and np.all(new[4:] < 1.0)
