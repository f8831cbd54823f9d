"""Host-side pieces of the training path (no GPU): the equation dataset the
training benchmark and the grok evaluation feed (src/gpt/grokking.rs:116-258)
and the AdamW defaults (src/gpt/config.rs:258-276), through the C ABI.

The dataset is checked against the oracle's restatement, which the published
step-0 cross-entropies pin (tests/test_oracle.py), for every operation; the
split sizes are the published 4704 / 4705 (docs/grokking.md:14-15).
"""
import ctypes

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
