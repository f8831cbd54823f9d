"""GPU: generate's on-device sampler against the oracle's sequential f32 sampler.

The device decides temperature sampling in parallel (exact f64 prefix sums
and rounding-error bounds) and falls back to the sequential f32 process only
on near-ties; it must return exactly the reference's token
(src/gpt/gpu.rs:2028-2049) for the same f32 logits and SplitMix64 state.  The
states are chosen here so the draw u lands exactly on, or one f32 step either
side of, CDF boundaries, which forces both the fallback and the boundary
handling; random rows cover the common path.  Vocabularies up to 1024 run
the one-wave sampler (the persistent decode's), larger ones the workgroup
sampler, and V above its LDS row cap its global-memory path.
"""
import numpy as np
import pytest

import grokking_abmod_amd as G
import oracle_lib as O

pytestmark = pytest.mark.gpu

state_for_unit = O.state_for_unit


def oracle_sample(rows, temperature, states):
    tokens, out = [], []
    for row, st in zip(rows, states):
        t, s = O.sample(row, temperature, int(st))
        tokens.append(t)
        out.append(s)
    return np.array(tokens, dtype=np.uint32), np.array(out, dtype=np.uint64)


def check(rows, temperature, states):
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    got, got_states = G.sample_logits(rows, temperature, np.array(states, dtype=np.uint64))
    want, want_states = oracle_sample(rows, temperature, states)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[0]}: got {got[bad[0]]}, want {want[bad[0]]}"
    assert np.array_equal(got_states, want_states)


def test_state_inversion_gives_requested_draw():
    for k in (0, 1, 1 << 22, (1 << 24) - 1, 12345678):
        assert O.rng_unit_at(state_for_unit(k), 1) == k / 16777216.0


def test_exact_cdf_boundaries_with_equal_logits():
    # Four equal logits: p = 1 each, S = 4, so u = j/4 puts u*S exactly on a CDF
    # boundary; one f32 step either side decides the other way.
    rows, states = [], []
    for j in (1, 2, 3):
        for dk in (-1, 0, 1):
            rows.append(np.full(4, 0.5, np.float32))
            states.append(state_for_unit(j * (1 << 22) + dk))
    for T in (1.0, 0.5):
        check(rows, T, states)


def test_near_ties_on_random_rows():
    # u placed on (and one step either side of) the f32 CDF value of a chosen
    # token, as the sequential process computes it.
    rng = np.random.default_rng(21)
    rows, states = [], []
    for trial in range(300):
        V = int(rng.choice([2, 3, 5, 17, 64, 99, 256]))
        T = 1.0
        row = (rng.normal(size=V) * 2).astype(np.float32)
        p = np.exp(((row - row.max()) / np.float32(T)).astype(np.float32)).astype(np.float32)
        S = np.float32(0)
        for v in p:
            S = np.float32(S + v)
        target = int(rng.integers(0, V))
        cum = float(np.cumsum(p.astype(np.float64))[target])
        k = int(round(cum / float(S) * (1 << 24)))
        for dk in (-1, 0, 1):
            kk = min(max(k + dk, 0), (1 << 24) - 1)
            rows.append(np.pad(row, (0, 256 - V), constant_values=np.float32(-1e30))[:V])
            states.append(state_for_unit(kk))
    by_len = {}
    for r, st in zip(rows, states):
        by_len.setdefault(len(r), ([], []))
        by_len[len(r)][0].append(r)
        by_len[len(r)][1].append(st)
    for V, (rs, sts) in by_len.items():
        check(np.stack(rs), 1.0, sts)


@pytest.mark.parametrize("V", [2, 7, 64, 99, 256, 1000, 5000])
@pytest.mark.parametrize("T", [0.0, 0.3, 1.0, 2.5])
def test_random_rows(V, T):
    rng = np.random.default_rng(V * 7 + int(T * 10))
    rows = (rng.normal(size=(64, V)) * 3).astype(np.float32)
    rows[::7, :] = rows[::7, :1]  # all-equal rows: greedy takes token 0
    states = rng.integers(0, 2**63, size=64, dtype=np.int64).astype(np.uint64)
    check(rows, T, states)


def test_nonfinite_rows_are_reported():
    rows = np.zeros((2, 8), np.float32)
    rows[1, 3] = np.nan
    with pytest.raises(G.MeshGptError) as info:
        G.sample_logits(rows, 1.0, np.array([1, 2], np.uint64))
    assert info.value.status == G.MG_NONFINITE


def _host_expf():
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    return libm.expf


def test_device_expf_matches_c_library():
    """The sampler's p_i = exp((l - max) / T) must be the reference's f32::exp,
    which is the C library's expf.  Special values, the underflow and
    denormal range, a fine grid and random inputs are compared bit for bit.
    Two inputs are rounded differently by glibc's build for hosts without
    FMA; they are skipped when this host's expf is that build."""
    expf = _host_expf()
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 88.0, 88.72283, 88.72284, -87.33655, -88.0, -100.0,
                        -103.27893, -103.972, -103.97208, -103.9721, -104.0, -120.0, 1e-30, -1e-30,
                        float.fromhex("0x1.04845ep+5"), -float.fromhex("0x1.f8cbb2p+5")], dtype=np.float32)
    grid = -np.arange(0, 110 * 1024, dtype=np.float32) / np.float32(1024.0)
    bits = rng.integers(0x80000000, 0xC2D00000, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([special, grid, bits.view(np.float32), rng.uniform(-110, 90, 200_000).astype(np.float32)])
    got = G.device_expf(x)
    want = np.array([expf(float(v)) for v in x], dtype=np.float32)
    differ = got.view(np.uint32) != want.view(np.uint32)
    differ &= ~(np.isnan(got) & np.isnan(want))
    non_fma_pair = {np.float32(float.fromhex("0x1.04845ep+5")).view(np.uint32),
                    np.float32(-float.fromhex("0x1.f8cbb2p+5")).view(np.uint32)}
    left = [hex(int(v)) for v in x[differ].view(np.uint32) if int(v) not in {int(u) for u in non_fma_pair}]
    assert not left, f"device expf differs from the C library at {left[:8]}"
