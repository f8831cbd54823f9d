"""Python binding of libmeshgpt.so, the MI355X Mesh GPT generate path.

A thin ctypes layer over the C ABI in include/meshgpt.h, mirroring the
reference's inference API (src/gpt/gpu.rs:1693-2092: ``SpecializedMeshGpt``)
and its host types (``GptConfig``, ``Checkpoint``).  The product is the native
library; this module only marshals arrays.  Importing it fails loudly when the
library has not been built: there is no fallback implementation.
"""
import ctypes
import os

import numpy as np

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PACKAGE_DIR, "libmeshgpt.so")
CLI_PATH = os.path.join(PACKAGE_DIR, "mesh-gpt")

MG_OK, MG_INVALID_ARGUMENT, MG_OUT_OF_MEMORY, MG_DEVICE_ERROR, MG_NONFINITE, MG_IO, MG_UNSUPPORTED = range(7)

# Every function include/meshgpt.h declares.
EXPORTS = (
    "mg_last_error", "mg_config_default", "mg_config_validate", "mg_parameter_count",
    "mg_initial_parameters", "mg_normal_parameters", "mg_token_codes", "mg_model_create", "mg_model_destroy",
    "mg_model_config", "mg_parameters", "mg_set_parameters", "mg_logits", "mg_token_embeddings",
    "mg_hidden_states", "mg_generate", "mg_generate_text", "mg_prefill", "mg_decode",
    "mg_decode_rewind", "mg_last_call_ms", "mg_decode_profiled", "mg_decode_traced", "mg_sequence_length", "mg_read_tokens", "mg_last_logits",
    "mg_model_stream", "mg_checkpoint_load", "mg_checkpoint_info", "mg_checkpoint_characters",
    "mg_checkpoint_parameters", "mg_checkpoint_free", "mg_checkpoint_save", "mg_copy_bandwidth",
    "mg_tokenizer_from_text", "mg_tokenizer_encode", "mg_tokenizer_decode", "mg_sample_logits", "mg_sample_logits_noalloc", "mg_expf",
    "mg_adamw_default", "mg_cross_entropy", "mg_loss_and_gradient", "mg_train_batch",
    "mg_equation_split", "mg_equation_batch", "mg_text_batch",
)

IGNORE_TARGET = 0xFFFFFFFF  # MG_IGNORE_TARGET (src/gpt/mod.rs:26)


class AdamW(ctypes.Structure):
    """mg_adamw: AdamWOptions (src/gpt/config.rs:258-276), reference defaults."""

    _fields_ = [(name, ctypes.c_float) for name in ("learning_rate", "weight_decay", "beta1", "beta2", "epsilon")]

    def __init__(self, **overrides):
        super().__init__()
        lib().mg_adamw_default(ctypes.byref(self))
        for key, value in overrides.items():
            if key not in dict(self._fields_):
                raise TypeError(f"unknown AdamW field {key}")
            setattr(self, key, float(value))


class GptConfig(ctypes.Structure):
    """mg_config: GptConfig (src/gpt/config.rs:21-56) in checkpoint field order."""

    _fields_ = [(name, ctypes.c_uint32) for name in (
        "vocab_size", "context", "width", "heads", "layers", "attention_mesh_depth",
        "ffn_mesh_depth", "embedding", "connectivity", "long_context", "rope", "qk_norm", "xsa",
        "form", "order", "frequency", "harmonics")] + [("overlap", ctypes.c_float)] + [
        (name, ctypes.c_uint32) for name in ("normalization", "frozen", "preserve_features", "modulus")] + [
        ("seed", ctypes.c_uint64)]

    def __init__(self, **overrides):
        super().__init__()
        lib().mg_config_default(ctypes.byref(self))
        for key, value in overrides.items():
            if key not in dict(self._fields_):
                raise TypeError(f"unknown GptConfig field {key}")
            setattr(self, key, float(value) if key == "overlap" else int(value))

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}

    def __repr__(self):
        return "GptConfig(" + ", ".join(f"{k}={v}" for k, v in self.as_dict().items()) + ")"

    def __eq__(self, other):
        return isinstance(other, GptConfig) and self.as_dict() == other.as_dict()


class MeshGptError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(message)
        self.status = status
        self.message = message


_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_szp = ctypes.POINTER(ctypes.c_size_t)
_cfgp = ctypes.POINTER(GptConfig)
_lib = None


def lib():
    """The loaded libmeshgpt.so; raises ImportError when it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                          "(or make -C grokking_abmod_amd/csrc)")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, i, u64, f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64, ctypes.c_float
    sigs = {
        "mg_last_error": (ctypes.c_char_p, []),
        "mg_config_default": (None, [_cfgp]),
        "mg_config_validate": (i, [_cfgp]),
        "mg_parameter_count": (i, [_cfgp, _szp]),
        "mg_initial_parameters": (i, [_cfgp, u64, _f32p, sz]),
        "mg_normal_parameters": (i, [_cfgp, u64, f, _f32p, sz]),
        "mg_token_codes": (i, [_cfgp, _f32p, sz]),
        "mg_model_create": (i, [i, _cfgp, u64, sz, ctypes.POINTER(vp)]),
        "mg_model_destroy": (None, [vp]),
        "mg_model_config": (i, [vp, _cfgp]),
        "mg_parameters": (i, [vp, _f32p, sz]),
        "mg_set_parameters": (i, [vp, _f32p, sz]),
        "mg_logits": (i, [vp, _u32p, sz, sz, i, _f32p, sz]),
        "mg_token_embeddings": (i, [vp, _f32p, sz]),
        "mg_hidden_states": (i, [vp, _u32p, sz, sz, _f32p, sz]),
        "mg_generate": (i, [vp, _u32p, sz, sz, sz, f, u64, _u32p]),
        "mg_generate_text": (i, [vp, _u32p, sz, ctypes.c_char_p, sz, f, u64, ctypes.c_char_p, sz, _szp]),
        "mg_prefill": (i, [vp, _u32p, sz, sz, f, u64, sz]),
        "mg_decode": (i, [vp, sz]),
        "mg_decode_rewind": (i, [vp]),
        "mg_last_call_ms": (i, [vp, ctypes.POINTER(ctypes.c_float)]),
        "mg_decode_profiled": (i, [vp, sz, _f32p, sz]),
        "mg_decode_traced": (i, [vp, sz, ctypes.POINTER(ctypes.c_uint64), sz]),
        "mg_sequence_length": (i, [vp, _szp]),
        "mg_read_tokens": (i, [vp, _u32p, sz, sz]),
        "mg_last_logits": (i, [vp, _f32p, sz]),
        "mg_model_stream": (vp, [vp]),
        "mg_checkpoint_load": (i, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "mg_checkpoint_info": (i, [vp, _cfgp, _szp, _szp]),
        "mg_checkpoint_characters": (i, [vp, _u32p, sz]),
        "mg_checkpoint_parameters": (i, [vp, _f32p, sz]),
        "mg_checkpoint_free": (None, [vp]),
        "mg_checkpoint_save": (i, [ctypes.c_char_p, _cfgp, _u32p, sz, _f32p, sz]),
        "mg_copy_bandwidth": (i, [i, sz, i, ctypes.POINTER(ctypes.c_double)]),
        "mg_tokenizer_from_text": (i, [ctypes.c_char_p, sz, _u32p, sz, _szp]),
        "mg_tokenizer_encode": (i, [_u32p, sz, ctypes.c_char_p, sz, _u32p, sz, _szp]),
        "mg_tokenizer_decode": (i, [_u32p, sz, _u32p, sz, ctypes.c_char_p, sz, _szp]),
        "mg_sample_logits": (i, [i, _f32p, sz, sz, f, ctypes.POINTER(ctypes.c_uint64), _u32p]),
        "mg_sample_logits_noalloc": (i, [i, vp, sz, sz, f, vp, vp, vp, vp]),
        "mg_expf": (i, [i, _f32p, sz, _f32p]),
        "mg_adamw_default": (None, [vp]),
        "mg_cross_entropy": (i, [vp, _u32p, _u32p, sz, sz, ctypes.POINTER(ctypes.c_double)]),
        "mg_loss_and_gradient": (i, [vp, _u32p, _u32p, sz, sz, ctypes.POINTER(ctypes.c_double), _f32p, sz]),
        "mg_train_batch": (i, [vp, _u32p, _u32p, sz, sz, vp, ctypes.POINTER(ctypes.c_double)]),
        "mg_equation_split": (i, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double, u64, _szp, _szp]),
        "mg_equation_batch": (i, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double, u64, i, _szp, sz, _u32p,
                                  _u32p]),
        "mg_text_batch": (i, [_u32p, sz, _cfgp, i, sz, sz, u64, _u32p, _u32p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(status):
    if status != MG_OK:
        raise MeshGptError(status, lib().mg_last_error().decode("utf-8", "replace"))


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a, kind):
    return a.ctypes.data_as(kind)


def validate(config):
    _check(lib().mg_config_validate(ctypes.byref(config)))


def parameter_count(config):
    n = ctypes.c_size_t()
    _check(lib().mg_parameter_count(ctypes.byref(config), ctypes.byref(n)))
    return n.value


def initial_parameters(config, seed):
    out = np.empty(parameter_count(config), dtype=np.float32)
    _check(lib().mg_initial_parameters(ctypes.byref(config), seed, _p(out, _f32p), out.size))
    return out


def normal_parameters(config, seed, sigma=0.5):
    """mg_normal_parameters: N(0, sigma^2) weights, the reference's Box-Muller
    draw on Random::new(seed) (src/simple/numerical.rs:163-167)."""
    out = np.empty(parameter_count(config), dtype=np.float32)
    _check(lib().mg_normal_parameters(ctypes.byref(config), seed, sigma, _p(out, _f32p), out.size))
    return out


def token_codes(config):
    out = np.empty((config.vocab_size, config.width), dtype=np.float32)
    _check(lib().mg_token_codes(ctypes.byref(config), _p(out, _f32p), out.size))
    return out


def copy_bandwidth(nbytes, iters=20, device=0):
    """Read+write GB/s of the library's plain copy kernel (calibration_copy)."""
    gbps = ctypes.c_double()
    _check(lib().mg_copy_bandwidth(device, nbytes, iters, ctypes.byref(gbps)))
    return gbps.value


def sample_logits(logits, temperature, rng_states, device=0):
    """generate's sampler on the device for rows of f32 logits; returns
    (tokens, advanced rng states)."""
    logits = _f32(np.atleast_2d(logits))
    states = np.ascontiguousarray(rng_states, dtype=np.uint64).copy()
    rows, vocab = logits.shape
    out = np.empty(rows, dtype=np.uint32)
    _check(lib().mg_sample_logits(device, _p(logits, _f32p), rows, vocab, temperature,
                                  states.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), _p(out, _u32p)))
    return out, states


def sample_logits_noalloc(logits_ptr, rows, vocab, temperature, rng_ptr, tokens_ptr, nonfinite_ptr, stream=None,
                          device=0):
    """mg_sample_logits_noalloc on device pointers (ints); enqueued on `stream`."""
    _check(lib().mg_sample_logits_noalloc(device, logits_ptr, rows, vocab, temperature, rng_ptr, tokens_ptr,
                                          nonfinite_ptr, stream))


def device_expf(x, device=0):
    """The sampler's f32 exp evaluated on the device."""
    x = _f32(np.ravel(x))
    out = np.empty_like(x)
    _check(lib().mg_expf(device, _p(x, _f32p), x.size, _p(out, _f32p)))
    return out


def calibration_copy(nbytes, device=0):
    """One warm-up and one timed launch of calibration_copy over nbytes."""
    return copy_bandwidth(nbytes, 1, device)


def equation_split(modulus=97, operation=0, train_fraction=0.5, seed=7):
    """EquationDataset::new (grokking.rs:128-186): (training, validation) sizes."""
    a, b = ctypes.c_size_t(), ctypes.c_size_t()
    _check(lib().mg_equation_split(modulus, operation, train_fraction, seed, ctypes.byref(a), ctypes.byref(b)))
    return a.value, b.value


def equation_batch(indices, validation=False, modulus=97, operation=0, train_fraction=0.5, seed=7):
    """EquationDataset::batch (grokking.rs:225-258): (inputs, targets), 4 rows an equation."""
    idx = np.ascontiguousarray(indices, dtype=np.uintp).reshape(-1)
    inputs = np.empty(4 * max(idx.size, 1), dtype=np.uint32)
    targets = np.empty_like(inputs)
    _check(lib().mg_equation_batch(modulus, operation, train_fraction, seed, int(validation),
                                   idx.ctypes.data_as(_szp), idx.size, _p(inputs, _u32p), _p(targets, _u32p)))
    return inputs[:4 * idx.size], targets[:4 * idx.size]


def text_batch(tokens, config, validation, sequence, batch, seed):
    """TextDataset::new + batch (src/gpt/text.rs:63-108): (inputs, targets) of
    batch windows of sequence tokens from the corpus's 90/10 split."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
    n = min(max(sequence * batch, 1), 131072)  # larger batches are rejected before anything is written
    inputs = np.empty(n, dtype=np.uint32)
    targets = np.empty_like(inputs)
    _check(lib().mg_text_batch(_p(t, _u32p), t.size, ctypes.byref(config), int(validation), sequence, batch, seed,
                               _p(inputs, _u32p), _p(targets, _u32p)))
    return inputs[:sequence * batch], targets[:sequence * batch]


class MeshGpt:
    """SpecializedMeshGpt (src/gpt/gpu.rs:1693-2092) on one MI355X."""

    def __init__(self, device, config, seed, max_batch=1):
        handle = ctypes.c_void_p()
        _check(lib().mg_model_create(device, ctypes.byref(config), seed, max_batch, ctypes.byref(handle)))
        self._h = handle
        self._config = GptConfig(**config.as_dict())
        self._batch = 0

    def close(self):
        if getattr(self, "_h", None):
            lib().mg_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def config(self):
        out = GptConfig()
        _check(lib().mg_model_config(self._h, ctypes.byref(out)))
        return out

    def parameters(self):
        out = np.empty(parameter_count(self._config), dtype=np.float32)
        _check(lib().mg_parameters(self._h, _p(out, _f32p), out.size))
        return out

    def set_parameters(self, values):
        values = _f32(values)
        _check(lib().mg_set_parameters(self._h, _p(values, _f32p), values.size))

    def logits(self, tokens, sequence, last_only=False):
        tokens = _u32(tokens).reshape(-1)
        rows = tokens.size // sequence if (last_only and sequence) else tokens.size
        out = np.empty((max(rows, 1), self._config.vocab_size), dtype=np.float32)
        _check(lib().mg_logits(self._h, _p(tokens, _u32p), tokens.size, sequence, int(last_only),
                               _p(out, _f32p), out.size))
        return out[:rows]

    def cross_entropy(self, inputs, targets, sequence):
        """gpu.rs:1915-1929: mean next-token loss over supervised rows."""
        inputs, targets = _u32(inputs).reshape(-1), _u32(targets).reshape(-1)
        if inputs.size != targets.size:
            raise MeshGptError(MG_INVALID_ARGUMENT, "inputs and targets must have equal lengths")
        loss = ctypes.c_double()
        _check(lib().mg_cross_entropy(self._h, _p(inputs, _u32p), _p(targets, _u32p), inputs.size, sequence,
                                      ctypes.byref(loss)))
        return loss.value

    def loss_and_gradient(self, inputs, targets, sequence):
        """gpu.rs:1931-1946: (loss, gradient of every parameter)."""
        inputs, targets = _u32(inputs).reshape(-1), _u32(targets).reshape(-1)
        if inputs.size != targets.size:
            raise MeshGptError(MG_INVALID_ARGUMENT, "inputs and targets must have equal lengths")
        grad = np.empty(parameter_count(self._config), dtype=np.float32)
        loss = ctypes.c_double()
        _check(lib().mg_loss_and_gradient(self._h, _p(inputs, _u32p), _p(targets, _u32p), inputs.size, sequence,
                                          ctypes.byref(loss), _p(grad, _f32p), grad.size))
        return loss.value, grad

    def train_batch(self, inputs, targets, sequence, options=None):
        """gpu.rs:1950-2003: the loss before one AdamW update."""
        inputs, targets = _u32(inputs).reshape(-1), _u32(targets).reshape(-1)
        if inputs.size != targets.size:
            raise MeshGptError(MG_INVALID_ARGUMENT, "inputs and targets must have equal lengths")
        options = AdamW() if options is None else options
        loss = ctypes.c_double()
        _check(lib().mg_train_batch(self._h, _p(inputs, _u32p), _p(targets, _u32p), inputs.size, sequence,
                                    ctypes.byref(options), ctypes.byref(loss)))
        return loss.value

    def token_embeddings(self):
        out = np.empty((self._config.vocab_size, self._config.width), dtype=np.float32)
        _check(lib().mg_token_embeddings(self._h, _p(out, _f32p), out.size))
        return out

    def hidden_states(self, tokens, sequence):
        tokens = _u32(tokens).reshape(-1)
        out = np.empty((max(tokens.size, 1), self._config.width), dtype=np.float32)
        _check(lib().mg_hidden_states(self._h, _p(tokens, _u32p), tokens.size, sequence,
                                      _p(out, _f32p), out.size))
        return out[:tokens.size]

    def generate_tokens(self, prompts, count, temperature, seed):
        prompts = _u32(np.atleast_2d(prompts))
        batch, length = prompts.shape
        self._batch = batch
        out = np.empty((batch, length + count), dtype=np.uint32)
        _check(lib().mg_generate(self._h, _p(prompts, _u32p), batch, length, count, temperature, seed,
                                 _p(out, _u32p)))
        return out

    def generate(self, characters, prompt, count, temperature, seed):
        chars = _u32([ord(c) if isinstance(c, str) else c for c in characters])
        data = prompt.encode("utf-8")
        capacity = 4 * (len(prompt) + count) + 16
        buf = ctypes.create_string_buffer(capacity)
        written = ctypes.c_size_t()
        _check(lib().mg_generate_text(self._h, _p(chars, _u32p), chars.size, data, count, temperature,
                                      seed, buf, capacity, ctypes.byref(written)))
        return buf.raw[:written.value].decode("utf-8")

    def prefill(self, prompts, temperature, seed, reserve=0):
        prompts = _u32(np.atleast_2d(prompts))
        batch, length = prompts.shape
        self._batch = batch
        _check(lib().mg_prefill(self._h, _p(prompts, _u32p), batch, length, temperature, seed, reserve))

    def decode(self, steps):
        _check(lib().mg_decode(self._h, steps))

    def last_call_ms(self):
        """Kernel time of the last logits / hidden_states / prefill call, or
        of the last persistent decode launch (ms)."""
        ms = ctypes.c_float()
        _check(lib().mg_last_call_ms(self._h, ctypes.byref(ms)))
        return ms.value

    def rewind(self):
        """Back to the decode state the last prefill left (mg_decode_rewind)."""
        _check(lib().mg_decode_rewind(self._h))

    def decode_profiled(self, steps):
        out = np.empty(steps * self._config.layers, dtype=np.float32)
        _check(lib().mg_decode_profiled(self._h, steps, _p(out, _f32p), out.size))
        return out

    def decode_traced(self, steps):
        """Persistent decode of `steps` steps with its timeline: an array
        [blocks, steps, layers + 1, 2] of 100 MHz wall-clock stamps (ready,
        published); blocks are 3*batch mesh teams, then batch*heads attention
        blocks."""
        c = self._config
        batch = self._batch
        blocks = 3 * batch + batch * c.heads
        out = np.zeros((blocks, steps, c.layers + 1, 2), dtype=np.uint64)
        _check(lib().mg_decode_traced(self._h, steps, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), out.size))
        return out

    def sequence_length(self):
        n = ctypes.c_size_t()
        _check(lib().mg_sequence_length(self._h, ctypes.byref(n)))
        return n.value

    def read_tokens(self, batch, length=None):
        length = self.sequence_length() if length is None else length
        out = np.empty((batch, length), dtype=np.uint32)
        _check(lib().mg_read_tokens(self._h, _p(out, _u32p), batch, length))
        return out

    def last_logits(self, batch):
        out = np.empty((batch, self._config.vocab_size), dtype=np.float32)
        _check(lib().mg_last_logits(self._h, _p(out, _f32p), out.size))
        return out

    def stream(self):
        return lib().mg_model_stream(self._h)


class CharacterTokenizer:
    """CharacterTokenizer (src/gpt/text.rs:7-56): token id = index into the sorted
    unique characters of a text."""

    def __init__(self, characters):
        self.characters = [c if isinstance(c, str) else chr(c) for c in characters]
        self._chars = _u32([ord(c) for c in self.characters])

    @staticmethod
    def from_text(text):
        data = text.encode("utf-8")
        n = ctypes.c_size_t()
        _check(lib().mg_tokenizer_from_text(data, len(data), None, 0, ctypes.byref(n)))
        out = np.empty(n.value, dtype=np.uint32)
        _check(lib().mg_tokenizer_from_text(data, len(data), _p(out, _u32p), out.size, ctypes.byref(n)))
        return CharacterTokenizer([int(c) for c in out])

    def vocab_size(self):
        return len(self.characters)

    def encode(self, text):
        data = text.encode("utf-8")
        out = np.empty(max(len(data), 1), dtype=np.uint32)
        n = ctypes.c_size_t()
        _check(lib().mg_tokenizer_encode(_p(self._chars, _u32p), self._chars.size, data, len(data),
                                         _p(out, _u32p), out.size, ctypes.byref(n)))
        return out[:n.value]

    def decode(self, tokens):
        tokens = _u32(tokens).reshape(-1)
        capacity = 4 * tokens.size + 1
        buf = ctypes.create_string_buffer(capacity)
        written = ctypes.c_size_t()
        _check(lib().mg_tokenizer_decode(_p(self._chars, _u32p), self._chars.size, _p(tokens, _u32p),
                                         tokens.size, buf, capacity, ctypes.byref(written)))
        return buf.raw[:written.value].decode("utf-8")

    def __eq__(self, other):
        return isinstance(other, CharacterTokenizer) and self.characters == other.characters


class Checkpoint:
    """Checkpoint (src/gpt/checkpoint.rs:14-192): config, tokenizer characters, weights."""

    def __init__(self, config, characters, parameters):
        self.config = config
        self.characters = list(characters)
        self.parameters = _f32(parameters)

    @staticmethod
    def load(path):
        handle = ctypes.c_void_p()
        _check(lib().mg_checkpoint_load(os.fsencode(path), ctypes.byref(handle)))
        try:
            config = GptConfig()
            vocab, count = ctypes.c_size_t(), ctypes.c_size_t()
            _check(lib().mg_checkpoint_info(handle, ctypes.byref(config), ctypes.byref(vocab),
                                            ctypes.byref(count)))
            chars = np.empty(vocab.value, dtype=np.uint32)
            params = np.empty(count.value, dtype=np.float32)
            _check(lib().mg_checkpoint_characters(handle, _p(chars, _u32p), chars.size))
            _check(lib().mg_checkpoint_parameters(handle, _p(params, _f32p), params.size))
        finally:
            lib().mg_checkpoint_free(handle)
        return Checkpoint(config, [int(c) for c in chars], params)

    def save(self, path):
        chars = _u32([ord(c) if isinstance(c, str) else c for c in self.characters])
        _check(lib().mg_checkpoint_save(os.fsencode(path), ctypes.byref(self.config), _p(chars, _u32p),
                                        chars.size, _p(self.parameters, _f32p), self.parameters.size))


_MASK64 = (1 << 64) - 1


def random_prompts(vocab_size, batch, length, seed=7):
    """Uniform token ids as the synthetic workloads draw them: Random::new(seed)
    (SplitMix64, src/mesh.rs:256-274) and index(vocab_size) with its rejection
    threshold (mesh.rs:277-288), sequence b drawn after sequence b-1; a
    (batch, length) uint32 array.  The CLI's --random-prompt draws the same."""
    state = seed & _MASK64
    bound = int(vocab_size)
    threshold = ((1 << 64) - bound) % bound
    out = np.empty((batch, length), dtype=np.uint32)
    for b in range(batch):
        for i in range(length):
            while True:
                state = (state + 0x9E3779B97F4A7C15) & _MASK64
                z = state
                z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
                z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
                z ^= z >> 31
                if z >= threshold:
                    out[b, i] = z % bound
                    break
    return out


def named_config(name):
    """The synthetic workloads of the benchmark (butterfly meshes, defaults otherwise)."""
    table = {
        "tiny": dict(vocab_size=64, width=128, heads=4, layers=2, attention_mesh_depth=7,
                     ffn_mesh_depth=7, context=256, connectivity=1),
        "symbolic": dict(vocab_size=99, width=128, heads=4, layers=2, attention_mesh_depth=4,
                         ffn_mesh_depth=6, context=4, connectivity=0),
        "mid": dict(vocab_size=256, width=512, heads=8, layers=6, attention_mesh_depth=9,
                    ffn_mesh_depth=9, context=1024, connectivity=1),
        "long": dict(vocab_size=256, width=512, heads=8, layers=4, attention_mesh_depth=9,
                     ffn_mesh_depth=9, context=8448, connectivity=1, long_context=1),
        "high": dict(vocab_size=256, width=1024, heads=16, layers=12, attention_mesh_depth=10,
                     ffn_mesh_depth=10, context=2048, connectivity=1),
    }
    return GptConfig(**table[name])
