"""ctypes loader for the CPU checker in oracle/ (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "_build", "liboracle.so")

_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_szp = ctypes.POINTER(ctypes.c_size_t)


class OgConfig(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint32) for name in (
        "vocab_size", "context", "width", "heads", "layers",
        "attention_mesh_depth", "ffn_mesh_depth", "embedding", "connectivity",
        "rope", "qk_norm", "xsa", "form", "order", "frequency", "harmonics")] + [
        ("overlap", ctypes.c_float)] + [(name, ctypes.c_uint32) for name in (
            "normalization", "frozen", "preserve_features", "modulus")] + [("seed", ctypes.c_uint64)]


def config(vocab_size=32, context=32, width=32, heads=4, layers=2, attention_mesh_depth=4,
           ffn_mesh_depth=6, embedding=0, connectivity=0, rope=1, qk_norm=1, xsa=1, form=0, order=0,
           frequency=1, harmonics=1, overlap=0.0, normalization=0, frozen=0, preserve_features=0, modulus=0,
           seed=0):
    """GptConfig::default() (reference src/gpt/config.rs:38-55, geometry.rs:66-81)
    with overrides."""
    return OgConfig(vocab_size, context, width, heads, layers, attention_mesh_depth,
                    ffn_mesh_depth, embedding, connectivity, rope, qk_norm, xsa, form, order,
                    frequency, harmonics, overlap, normalization, frozen, preserve_features, modulus,
                    seed)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        L = ctypes.CDLL(LIB_PATH)
        cp = ctypes.POINTER(OgConfig)
        sigs = {
            "og_rng_next": (ctypes.c_uint64, [_u64p]),
            "og_rng_unit": (ctypes.c_float, [_u64p]),
            "og_rng_index": (ctypes.c_uint64, [_u64p, ctypes.c_uint64]),
            "og_validate": (ctypes.c_int, [cp, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]),
            "og_parameter_count": (ctypes.c_size_t, [cp]),
            "og_embedding_parameter_count": (ctypes.c_size_t, [cp]),
            "og_group_offsets": (None, [cp, _szp]),
            "og_constrained_range": (None, [cp, ctypes.c_size_t, _szp, _szp]),
            "og_stride": (ctypes.c_uint32, [cp, ctypes.c_uint32]),
            "og_initialize": (None, [cp, ctypes.c_uint64, _f32p]),
            "og_initialize_normal": (None, [cp, ctypes.c_uint64, ctypes.c_float, _f32p]),
            "cb_generate_f32": (ctypes.c_int, [cp, _f32p, _u32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                               ctypes.c_float, ctypes.c_uint64, ctypes.c_int, _u32p,
                                               ctypes.POINTER(ctypes.c_double)]),
            "og_token_codes": (None, [cp, _f32p]),
            "og_residue_permutation": (None, [ctypes.c_uint32, ctypes.c_uint64, _u32p]),
            "og_primitive_root": (ctypes.c_uint32, [ctypes.c_uint32]),
            "og_rmsnorm": (None, [_f64p, ctypes.c_size_t, ctypes.c_size_t, _f64p]),
            "og_rotary": (None, [_f64p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _f64p]),
            "og_exclusive": (None, [_f64p, _f64p, ctypes.c_size_t, ctypes.c_size_t, _f64p]),
            "og_attention": (None, [_f64p, _f64p, _f64p, ctypes.c_size_t, ctypes.c_size_t,
                                    ctypes.c_size_t, ctypes.c_size_t, _f64p]),
            "og_mesh": (None, [_f64p, ctypes.c_size_t, ctypes.c_size_t, _f32p, ctypes.c_size_t,
                               ctypes.c_uint32, _f64p]),
            "og_token_embeddings": (ctypes.c_int, [cp, _f32p, _f64p]),
            "og_logits": (ctypes.c_int, [cp, _f32p, _u32p, ctypes.c_size_t, ctypes.c_size_t, _f64p]),
            "og_hidden_states": (ctypes.c_int, [cp, _f32p, _u32p, ctypes.c_size_t, ctypes.c_size_t,
                                                _f64p]),
            "og_cross_entropy": (ctypes.c_int, [cp, _f32p, _u32p, _u32p, ctypes.c_size_t,
                                                ctypes.c_size_t, _f64p]),
            "og_generate": (ctypes.c_int, [cp, _f32p, _u32p, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_float, ctypes.c_uint64, _u32p]),
            "og_generate_cached": (ctypes.c_int, [cp, _f32p, _u32p, ctypes.c_size_t,
                                                  ctypes.c_size_t, ctypes.c_float, ctypes.c_uint64,
                                                  _u32p, _f32p]),
            "og_sample": (ctypes.c_uint32, [_f32p, ctypes.c_size_t, ctypes.c_float, _u64p]),
            "og_text_batch": (ctypes.c_int, [_u32p, ctypes.c_size_t, ctypes.c_int, ctypes.c_size_t,
                                             ctypes.c_size_t, ctypes.c_uint64, _u32p, _u32p]),
            "og_equations": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double,
                                            ctypes.c_uint64, _u32p, _u32p, _u32p, _szp, _szp]),
            "og_row_metrics": (ctypes.c_double, [_f32p, ctypes.c_size_t, ctypes.c_size_t, _szp]),
            "og_loss_and_gradient": (ctypes.c_int, [cp, _f32p, _u32p, _u32p, ctypes.c_size_t,
                                                    ctypes.c_size_t, _f64p, _f64p]),
            "og_adam": (None, [_f32p, _f32p, _f32p, _f32p, ctypes.c_size_t, ctypes.c_float, ctypes.c_float,
                               ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                               ctypes.c_float]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a, kind):
    return a.ctypes.data_as(kind)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def validate(c, allow_long_context=False):
    buf = ctypes.create_string_buffer(256)
    rc = lib().og_validate(ctypes.byref(c), int(allow_long_context), buf, 256)
    return None if rc == 0 else buf.value.decode()


def parameter_count(c):
    return lib().og_parameter_count(ctypes.byref(c))


def group_offsets(c):
    out = np.zeros(1 + 5 * c.layers, dtype=np.uintp)
    lib().og_group_offsets(ctypes.byref(c), out.ctypes.data_as(_szp))
    return [int(x) for x in out]


def stride(c, layer):
    return lib().og_stride(ctypes.byref(c), layer)


def initialize(c, seed):
    out = np.zeros(parameter_count(c), dtype=np.float32)
    lib().og_initialize(ctypes.byref(c), seed, ptr(out, _f32p))
    return out


def initialize_normal(c, seed, sigma=0.5):
    out = np.zeros(parameter_count(c), dtype=np.float32)
    lib().og_initialize_normal(ctypes.byref(c), seed, sigma, ptr(out, _f32p))
    return out


def token_codes(c):
    out = np.zeros((c.vocab_size, c.width), dtype=np.float32)
    lib().og_token_codes(ctypes.byref(c), ptr(out, _f32p))
    return out


def rmsnorm(x, heads):
    x = f64(x)
    out = np.zeros_like(x)
    lib().og_rmsnorm(ptr(x, _f64p), x.size, heads, ptr(out, _f64p))
    return out


def rotary(x, heads, position):
    x = f64(x)
    out = np.zeros_like(x)
    lib().og_rotary(ptr(x, _f64p), x.size, heads, position, ptr(out, _f64p))
    return out


def exclusive(y, v, heads):
    y, v = f64(y), f64(v)
    out = np.zeros_like(y)
    lib().og_exclusive(ptr(y, _f64p), ptr(v, _f64p), y.size, heads, ptr(out, _f64p))
    return out


def attention(q, k, v, heads, sequence):
    q, k, v = f64(q), f64(k), f64(v)
    rows, width = q.shape
    out = np.zeros_like(q)
    lib().og_attention(ptr(q, _f64p), ptr(k, _f64p), ptr(v, _f64p), rows, width, heads, sequence,
                       ptr(out, _f64p))
    return out


def mesh(x, params, depth, connectivity):
    x = f64(x)
    params = f32(params)
    rows, width = x.shape
    out = np.zeros_like(x)
    lib().og_mesh(ptr(x, _f64p), rows, width, ptr(params, _f32p), depth, connectivity,
                  ptr(out, _f64p))
    return out


def token_embeddings(c, params):
    params = f32(params)
    out = np.zeros((c.vocab_size, c.width), dtype=np.float64)
    lib().og_token_embeddings(ctypes.byref(c), ptr(params, _f32p), ptr(out, _f64p))
    return out


def logits(c, params, tokens, sequence):
    params, tokens = f32(params), u32(tokens)
    out = np.zeros((tokens.size, c.vocab_size), dtype=np.float64)
    rc = lib().og_logits(ctypes.byref(c), ptr(params, _f32p), ptr(tokens, _u32p), tokens.size,
                         sequence, ptr(out, _f64p))
    if rc:
        raise ValueError("oracle rejected the token batch")
    return out


def hidden_states(c, params, tokens, sequence):
    params, tokens = f32(params), u32(tokens)
    out = np.zeros((tokens.size, c.width), dtype=np.float64)
    rc = lib().og_hidden_states(ctypes.byref(c), ptr(params, _f32p), ptr(tokens, _u32p),
                                tokens.size, sequence, ptr(out, _f64p))
    if rc:
        raise ValueError("oracle rejected the token batch")
    return out


def cross_entropy(c, params, inputs, targets, sequence):
    params, inputs, targets = f32(params), u32(inputs), u32(targets)
    out = ctypes.c_double()
    rc = lib().og_cross_entropy(ctypes.byref(c), ptr(params, _f32p), ptr(inputs, _u32p),
                                ptr(targets, _u32p), inputs.size, sequence, ctypes.byref(out))
    if rc:
        raise ValueError("oracle rejected the batch")
    return out.value


IGNORE = 0xFFFFFFFF  # IGNORE_TARGET (src/gpt/mod.rs:26)


def loss_and_gradient(c, params, inputs, targets, sequence):
    """(loss, gradient) of reference.rs:61-89 by the restated tape; raises
    ValueError with the oracle's status on a rejected batch."""
    params, inputs, targets = f32(params), u32(inputs), u32(targets)
    grad = np.zeros(parameter_count(c), dtype=np.float64)
    loss = ctypes.c_double()
    rc = lib().og_loss_and_gradient(ctypes.byref(c), ptr(params, _f32p), ptr(inputs, _u32p),
                                    ptr(targets, _u32p), inputs.size, sequence, ctypes.byref(loss),
                                    ptr(grad, _f64p))
    if rc:
        raise ValueError(f"oracle rejected the batch ({rc})")
    return loss.value, grad


class Adam:
    """AdamW state of the GPU path (gpu.rs:1366-1391,1971-2003): f32 moments and
    f32 running powers of the betas."""

    def __init__(self, params, learning_rate=0.003, weight_decay=0.01, beta1=0.9, beta2=0.999, epsilon=1e-8):
        self.value = f32(params).copy()
        self.m = np.zeros_like(self.value)
        self.v = np.zeros_like(self.value)
        self.opts = [np.float32(x) for x in (learning_rate, weight_decay, beta1, beta2, epsilon)]
        self.p1 = np.float32(1.0)
        self.p2 = np.float32(1.0)

    def step(self, gradient, skip=0):
        """One update with `gradient` (cast to f32); the first `skip` parameters
        (a frozen embedding group) are left alone."""
        lr, wd, b1, b2, eps = self.opts
        self.p1 = np.float32(self.p1 * b1)
        self.p2 = np.float32(self.p2 * b2)
        g = f32(gradient)
        n = self.value.size - skip
        lib().og_adam(ptr(self.value[skip:], _f32p), ptr(self.m[skip:], _f32p), ptr(self.v[skip:], _f32p),
                      ptr(g[skip:], _f32p), n, lr, wd, b1, b2, eps, np.float32(1.0) - self.p1,
                      np.float32(1.0) - self.p2)
        return self.value


def generate(c, params, prompt, count, temperature, seed, cached=False):
    params, prompt = f32(params), u32(prompt)
    out = np.zeros(prompt.size + count, dtype=np.uint32)
    if cached:
        rc = lib().og_generate_cached(ctypes.byref(c), ptr(params, _f32p), ptr(prompt, _u32p),
                                      prompt.size, count, temperature, seed, ptr(out, _u32p), None)
    else:
        rc = lib().og_generate(ctypes.byref(c), ptr(params, _f32p), ptr(prompt, _u32p),
                               prompt.size, count, temperature, seed, ptr(out, _u32p))
    if rc:
        raise ValueError("oracle rejected the generation request")
    return out


def cpu_generate_f32(c, params, prompts, steps, temperature, seed, threads):
    """The CPU baseline (cpu_f32_decode.c): KV-cached f32 decode of the
    (B, P) prompts on `threads` threads; returns (tokens B x (P + steps + 1),
    seconds of the decode steps)."""
    params, prompts = f32(params), np.ascontiguousarray(prompts, dtype=np.uint32)
    B, P = prompts.shape
    out = np.zeros((B, P + steps + 1), dtype=np.uint32)
    seconds = ctypes.c_double()
    rc = lib().cb_generate_f32(ctypes.byref(c), ptr(params, _f32p), ptr(prompts, _u32p), B, P, steps, temperature,
                               seed, threads, ptr(out, _u32p), ctypes.byref(seconds))
    if rc:
        raise ValueError("the CPU baseline does not take this shape")
    return out, seconds.value


def sample(logits_f32, temperature, rng_state):
    """Returns (token, new_rng_state)."""
    row = f32(logits_f32)
    state = ctypes.c_uint64(rng_state)
    token = lib().og_sample(ptr(row, _f32p), row.size, temperature, ctypes.byref(state))
    return int(token), state.value


def rng_unit_at(seed, k):
    """The k-th (1-based) Random::unit() draw of Random::new(seed)."""
    state = ctypes.c_uint64(seed)
    value = None
    for _ in range(k):
        value = lib().og_rng_unit(ctypes.byref(state))
    return value


def text_batch(tokens, validation, sequence, batch, seed):
    tokens = u32(tokens)
    x = np.zeros(sequence * batch, dtype=np.uint32)
    y = np.zeros(sequence * batch, dtype=np.uint32)
    rc = lib().og_text_batch(ptr(tokens, _u32p), tokens.size, int(validation), sequence, batch,
                             seed, ptr(x, _u32p), ptr(y, _u32p))
    if rc:
        raise ValueError("invalid dataset batch dimensions")
    return x, y


def equations(modulus=97, operation=0, train_fraction=0.5, seed=7):
    res = np.zeros(modulus, dtype=np.uint32)
    total = modulus * modulus
    train = np.zeros(3 * total, dtype=np.uint32)
    valid = np.zeros(3 * total, dtype=np.uint32)
    nt, nv = ctypes.c_size_t(), ctypes.c_size_t()
    rc = lib().og_equations(modulus, operation, train_fraction, seed, ptr(res, _u32p),
                            ptr(train, _u32p), ptr(valid, _u32p), ctypes.byref(nt), ctypes.byref(nv))
    if rc:
        raise ValueError("invalid equation dataset")
    return res, train[:3 * nt.value].reshape(-1, 3), valid[:3 * nv.value].reshape(-1, 3)


def row_metrics(row, target):
    row = f32(row)
    pred = ctypes.c_size_t()
    ce = lib().og_row_metrics(ptr(row, _f32p), row.size, target, ctypes.byref(pred))
    return ce, pred.value


def equation_inputs(residue_tokens, eqs, modulus=97):
    """EquationDataset::batch rows [res[a], op, res[b], '='] (grokking.rs:243-248)."""
    n = eqs.shape[0]
    x = np.empty((n, 4), dtype=np.uint32)
    x[:, 0] = residue_tokens[eqs[:, 0]]
    x[:, 1] = modulus
    x[:, 2] = residue_tokens[eqs[:, 1]]
    x[:, 3] = modulus + 1
    return x.reshape(-1), residue_tokens[eqs[:, 2]]


_MASK = (1 << 64) - 1
_GOLDEN = 0x9E3779B97F4A7C15
_C1, _C2 = 0xBF58476D1CE4E5B9, 0x94D049BB133111EB


def _unxorshift(y, s):
    x = y
    for _ in range(64 // s + 1):
        x = y ^ (x >> s)
    return x & _MASK


def state_for_unit(k):
    """A SplitMix64 state whose next Random::unit() draw is k / 2^24
    (src/mesh.rs:263-274), by inverting the output mix."""
    z = (k << 40) | 0x12345
    z = _unxorshift(z, 31)
    z = (z * pow(_C2, -1, 1 << 64)) & _MASK
    z = _unxorshift(z, 27)
    z = (z * pow(_C1, -1, 1 << 64)) & _MASK
    z = _unxorshift(z, 30)
    return (z - _GOLDEN) & _MASK
