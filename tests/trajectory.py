"""Token-trajectory parity against the oracle's generate loop.

The device's generated tokens must equal the oracle's (src/gpt/gpu.rs:2006-2053)
except where the decision was within the rounding of the two paths.  At the
first divergence the checker computes, on the same prefix, the oracle's f64
logits and the device's (a device re-prefill of the window), and the measured
error e = max |device - oracle| between them:

- greedy: the oracle's top-2 gap must be at most 2e (either order is then
  possible);
- temperature T: the draw u*S must lie within 2*expm1(2e'/T) + (V+2)*2^-23 of a
  CDF boundary (relative to the sum), e' = e plus the f32 rounding of the
  oracle logits: each p_i = exp((l_i - max)/T) moves by a factor within
  exp(+-2e'/T), so every normalised boundary moves by at most 2*expm1(2e'/T),
  and the f32 sums of the reference's sampler add at most (V+2)*2^-24 of the
  sum each.

A divergence that passes is legitimate; the oracle then continues from the
device's own prefix, with the generator state advanced by one draw per sampled
token (SplitMix64's state after n draws from seed s is s + n*0x9e3779b97f4a7c15,
src/mesh.rs:267-274), so every later token is checked too.
"""
import numpy as np

import oracle_lib as O

GOLDEN = 0x9E3779B97F4A7C15
MASK = (1 << 64) - 1


def sampling_margin(row, temperature, u):
    """Distance, relative to the sum, between u*sum and the nearest CDF boundary."""
    row = np.asarray(row, dtype=np.float64)
    p = np.exp((row - row.max()) / temperature)
    cdf = np.cumsum(p)
    return float(np.min(np.abs(cdf - u * cdf[-1])) / cdf[-1])


def sampling_bound(err, temperature, vocab):
    return 2.0 * np.expm1(2.0 * err / temperature) + (vocab + 2) * 2.0 ** -23


def check_trajectory(o, params, prompt, got, temperature, seed, device_logits, cached=True,
                     max_divergences=4, expected=None):
    """Checks a device trajectory `got` (prompt + generated) against the oracle.

    device_logits(prefix) returns the device's last-row logits for the window
    of `prefix` (the reference's window: its last `context` tokens).  Returns
    (number of tokens checked equal, number of legitimate divergences)."""
    prompt = np.asarray(prompt, dtype=np.uint32)
    got = np.asarray(got, dtype=np.uint32)
    P = len(prompt)
    assert np.array_equal(got[:P], prompt), "the prompt itself differs"
    count = len(got) - P
    if expected is None:
        expected = O.generate(o, params, prompt, count, temperature, seed, cached=cached)
    divergences = 0
    while True:
        diff = np.nonzero(got != expected)[0]
        if diff.size == 0:
            return len(got), divergences
        k = int(diff[0])
        window = got[:k][-o.context:]
        ref = O.logits(o, params, window, len(window))[-1]
        dev = np.asarray(device_logits(window), dtype=np.float64).reshape(-1)
        err = float(np.max(np.abs(dev - ref)))
        where = f"token {k} (step {k - P}): device {got[k]}, oracle {expected[k]}, logit error {err:.3g}"
        if temperature == 0.0:
            top = np.sort(ref)[-2:]
            assert top[1] - top[0] <= 2.0 * err, f"greedy {where}: top-2 gap {top[1] - top[0]:.3g}"
            next_seed = seed
        else:
            draws = k - P + 1
            u = O.rng_unit_at(seed, draws)
            ref32 = ref.astype(np.float32)
            err32 = err + float(np.max(np.abs(ref32.astype(np.float64) - ref)))
            margin = sampling_margin(ref32, temperature, u)
            bound = sampling_bound(err32, temperature, o.vocab_size)
            assert margin <= bound, f"sampled {where}: draw {margin:.3g} from a boundary, bound {bound:.3g}"
            next_seed = (seed + draws * GOLDEN) & MASK
        divergences += 1
        assert divergences <= max_divergences, f"more than {max_divergences} divergences, last at {where}"
        rest = O.generate(o, params, got[:k + 1], len(got) - k - 1, temperature, next_seed, cached=cached)
        expected = rest
