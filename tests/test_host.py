"""CPU tests of libmeshgpt.so's host side: no GPU call is made here.

Covers the C ABI surface (every symbol include/meshgpt.h declares is
exported), the host types that mirror the reference's Rust types -- GptConfig
validation (src/gpt/config.rs:144-228), layout and seeded initialisation
(config.rs:351-459), token codes (config.rs:552-591), CharacterTokenizer
(src/gpt/text.rs:7-56), Checkpoint MSHGPT07/08/09 (src/gpt/checkpoint.rs) -- and
the mesh-gpt CLI's host-only paths (help, init, argument errors).  Values are
compared with the oracle and with the reference's own KATs.
"""
import os
import re
import struct
import subprocess

import numpy as np
import pytest

import grokking_abmod_amd as G
import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "meshgpt.h")
DEMO = os.path.join(ROOT, "tests", "golden", "mesh-gpt-demo.txt")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mg_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 30
    lib = G.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The Python binding types every declared entry point, and nothing else.
    assert sorted(G.EXPORTS) == names


def test_default_config_is_reference_default():
    # config.rs:38-55
    c = G.GptConfig()
    assert c.as_dict() == dict(vocab_size=32, context=32, width=32, heads=4, layers=2, attention_mesh_depth=4,
                               ffn_mesh_depth=6, embedding=0, connectivity=0, long_context=0, rope=1, qk_norm=1,
                               xsa=1, form=0, order=0, frequency=1, harmonics=1, overlap=0.0, normalization=0,
                               frozen=0, preserve_features=0, modulus=0, seed=0)
    G.validate(c)
    assert G.parameter_count(c) == 3072


@pytest.mark.parametrize("kw,message", [
    (dict(vocab_size=1), "vocab_size must be in 2..65536"),
    (dict(vocab_size=65537), "vocab_size must be in 2..65536"),
    (dict(context=0), "context must be in 1..4096"),
    (dict(context=4097), "context must be in 1..4096"),
    (dict(width=1), "width must be in 2..4096"),
    (dict(width=4098), "width must be in 2..4096"),
    (dict(heads=3), "heads must be in 1..64 and divide width"),
    (dict(heads=0), "heads must be in 1..64 and divide width"),
    (dict(width=8, heads=8), "each attention head requires at least two channels"),
    (dict(width=6, heads=2), "slice RoPE requires an even number of channels per head"),
    (dict(layers=65), "layers must be in 1..64"),
    (dict(layers=0), "layers must be in 1..64"),
    (dict(ffn_mesh_depth=0), "mesh depths must be in 1..256"),
    (dict(attention_mesh_depth=257), "mesh depths must be in 1..256"),
])
def test_validation_messages_match_reference(kw, message):
    # config.rs:144-172 and its rejection KAT config.rs:720-776
    with pytest.raises(G.MeshGptError, match=re.escape(message)) as info:
        G.validate(G.GptConfig(**kw))
    assert info.value.status == G.MG_INVALID_ARGUMENT
    assert O.validate(O.config(**kw)) == message


GEOMETRY_BASE = dict(vocab_size=7, width=8, heads=2, layers=2, attention_mesh_depth=2, ffn_mesh_depth=2, embedding=1)


@pytest.mark.parametrize("kw,message", [
    (dict(form=5, overlap=-0.2), "equiangular embedding does not fit vocabulary 7, width 8, overlap -0.2"),
    (dict(form=5, overlap=1.1), "equiangular embedding does not fit vocabulary 7, width 8, overlap 1.1"),
    (dict(form=5, overlap=float("nan")), "embedding overlap must be finite; preserved features must fit width"),
    (dict(form=5, overlap=0.0, width=6, heads=1), "equiangular embedding does not fit vocabulary 7, width 6, overlap 0"),
    (dict(form=3, width=6, heads=1), "orthogonal embedding does not fit vocabulary 7, width 6, overlap 0"),
    (dict(form=7, width=2, heads=1, vocab_size=9), "hypercube embedding does not fit vocabulary 9, width 2, overlap 0"),
    (dict(form=8, vocab_size=257), "signed-permutations embedding does not fit vocabulary 257, width 8, overlap 0"),
    (dict(harmonics=0), "embedding frequency must be positive and harmonics in 1..width/2"),
    (dict(harmonics=5), "embedding frequency must be positive and harmonics in 1..width/2"),
    (dict(frequency=0), "embedding frequency must be positive and harmonics in 1..width/2"),
    (dict(preserve_features=9), "embedding overlap must be finite; preserved features must fit width"),
    (dict(preserve_features=1, normalization=1),
     "preserved coordinates require --embedding-norm none; full-vector normalization would rescale the "
     "protected feature"),
    (dict(order=1, modulus=4, vocab_size=6), "arithmetic embedding order requires a grok prime and vocabulary modulus+2"),
    (dict(order=1, modulus=5, vocab_size=8), "arithmetic embedding order requires a grok prime and vocabulary modulus+2"),
    (dict(order=2, modulus=5, form=1, width=4),
     "arithmetic circle/Fourier codes need extra coordinates for special symbols"),
    (dict(width=6, heads=2), "slice RoPE requires an even number of channels per head"),
])
def test_geometry_validation_messages_match_reference(kw, message):
    # geometry.rs:84-151 and config.rs:160 on the product and the oracle
    cfg = dict(GEOMETRY_BASE, **kw)
    with pytest.raises(G.MeshGptError, match=re.escape(message)):
        G.validate(G.GptConfig(**cfg))
    assert O.validate(O.config(**cfg)) == message


def test_rope_off_allows_odd_head_width_and_valid_geometries_pass():
    for kw in (dict(width=6, heads=2, rope=0), dict(form=4, width=6, heads=1), dict(form=5, overlap=1.0),
               dict(order=2, modulus=5, form=1, width=6, heads=3), dict(form=9), dict(preserve_features=8)):
        cfg = dict(GEOMETRY_BASE, **kw)
        G.validate(G.GptConfig(**cfg))
        assert O.validate(O.config(**cfg)) is None


GEOMETRY_CONFIGS = [
    dict(form=1), dict(form=2, harmonics=3, width=12), dict(form=3), dict(form=4), dict(form=5, overlap=0.25),
    dict(form=5, overlap=1.0), dict(form=6), dict(form=7), dict(form=8, vocab_size=200, width=8), dict(form=9),
    dict(form=9, seed=123456789012345), dict(form=1, order=1, modulus=5, seed=17),
    dict(form=2, order=2, modulus=5, seed=17, harmonics=2, width=12), dict(form=0, order=1, modulus=5, seed=3),
    dict(form=0, order=2, modulus=5, seed=3), dict(preserve_features=3), dict(normalization=2),
    dict(preserve_features=2, embedding=0), dict(form=3, embedding=0, normalization=1),
]


@pytest.mark.parametrize("kw", GEOMETRY_CONFIGS, ids=[str(i) for i in range(len(GEOMETRY_CONFIGS))])
def test_geometry_codes_and_initial_parameters_bit_equal_oracle(kw):
    # geometry.rs:186-325 codes and config.rs:416-459 initialisation (table
    # rows = codes for geometric forms, protected rows zeroed) on both sides.
    cfg = dict(GEOMETRY_BASE, **kw)
    g, o = G.GptConfig(**cfg), O.config(**cfg)
    assert np.array_equal(G.token_codes(g).view(np.uint32), O.token_codes(o).view(np.uint32))
    for seed in (0, 7):
        assert np.array_equal(G.initial_parameters(g, seed).view(np.uint32), O.initialize(o, seed).view(np.uint32))


def test_long_context_extension_is_opt_in():
    with pytest.raises(G.MeshGptError):
        G.validate(G.GptConfig(context=8448))
    G.validate(G.GptConfig(context=8448, long_context=1))
    with pytest.raises(G.MeshGptError):
        G.validate(G.GptConfig(context=65537, long_context=1))


@pytest.mark.parametrize("kw", [
    dict(),
    dict(vocab_size=26),
    dict(vocab_size=64, width=128, heads=4, layers=2, attention_mesh_depth=7, ffn_mesh_depth=7, connectivity=1),
    dict(vocab_size=256, width=512, heads=8, layers=6, attention_mesh_depth=9, ffn_mesh_depth=9, connectivity=1),
    dict(vocab_size=99, width=16, attention_mesh_depth=6, embedding=1),
    dict(vocab_size=99, width=16, attention_mesh_depth=6, embedding=1, connectivity=1),
    dict(vocab_size=7, width=6, heads=3),
])
def test_initial_parameters_and_codes_bit_equal_oracle(kw):
    # The product's seeded weights and token codes are exactly the oracle's
    # (config.rs:187-190, 416-459, 552-591), and the layout size is 2W(A+L(4A+F)).
    g, o = G.GptConfig(**kw), O.config(**kw)
    assert G.parameter_count(g) == O.parameter_count(o)
    for seed in (0, 7, 2**64 - 1):
        assert np.array_equal(G.initial_parameters(g, seed).view(np.uint32), O.initialize(o, seed).view(np.uint32))
    assert np.array_equal(G.token_codes(g), O.token_codes(o))


@pytest.mark.parametrize("kw", [
    dict(vocab_size=64, width=128, heads=4, layers=2, attention_mesh_depth=7, ffn_mesh_depth=7, connectivity=1),
    dict(vocab_size=256, width=512, heads=8, layers=6, attention_mesh_depth=9, ffn_mesh_depth=9, connectivity=1),
    dict(vocab_size=99, width=16, attention_mesh_depth=6, embedding=1),
    dict(vocab_size=16, width=32, heads=4, layers=2, preserve_features=3),
])
def test_normal_parameters_bit_equal_oracle(kw):
    # mg_normal_parameters (N(0, sigma^2) weights) equals the oracle's
    # restatement to the bit, for several seeds and sigmas.
    g, o = G.GptConfig(**kw), O.config(**kw)
    for seed, sigma in ((7, 0.5), (0, 1.0), (2**64 - 1, 0.125)):
        assert np.array_equal(G.normal_parameters(g, seed, sigma).view(np.uint32),
                              O.initialize_normal(o, seed, sigma).view(np.uint32))
    with pytest.raises(G.MeshGptError, match="finite nonnegative sigma"):
        G.normal_parameters(g, 7, -1.0)


def test_parameter_counts_of_the_benchmark_configs():
    # 2W(A + L(4A + F)) for the five workloads
    expected = dict(tiny=19712, symbolic=12288, mid=285696, long=193536, high=1249280)
    for name, count in expected.items():
        assert G.parameter_count(G.named_config(name)) == count


def test_random_prompts_are_reference_index_draws():
    # The synthetic prompts: Random::new(seed).index(V) (src/mesh.rs:277-288)
    # in sequence order, against the oracle's restatement of the generator.
    for vocab, batch, length, seed in ((256, 3, 17, 7), (64, 1, 16, 7), (99, 2, 5, 2**64 - 1), (3, 2, 40, 0)):
        got = G.random_prompts(vocab, batch, length, seed)
        state = O.ctypes.c_uint64(seed)
        want = [O.lib().og_rng_index(O.ctypes.byref(state), vocab) for _ in range(batch * length)]
        assert got.dtype == np.uint32 and got.shape == (batch, length)
        assert np.array_equal(got.ravel(), np.array(want, dtype=np.uint32))


# ---------------------------------------------------------------- tokenizer

def test_tokenizer_round_trip_and_errors():
    # text.rs:115-130
    text = "abc def\n" * 80
    t = G.CharacterTokenizer.from_text(text)
    assert t.characters == sorted(set(text))
    assert t.decode(t.encode(text)) == text
    with pytest.raises(G.MeshGptError, match="character '\\?' is outside the tokenizer vocabulary"):
        t.encode("?")
    with pytest.raises(G.MeshGptError, match="token ID is outside the tokenizer vocabulary"):
        t.decode([999])
    # Unicode scalars, not bytes; sorted by code point (a BTreeSet of char).
    u = G.CharacterTokenizer.from_text("héllo wörld ☃")
    assert u.characters == sorted(set("héllo wörld ☃"))
    assert u.decode(u.encode("wörld ☃")) == "wörld ☃"
    with pytest.raises(G.MeshGptError, match="tokenizer must contain 2..65536 unique characters"):
        G.CharacterTokenizer.from_text("aaaa")
    with pytest.raises(G.MeshGptError, match="tokenizer must contain 2..65536 unique characters"):
        G.CharacterTokenizer.from_text("")


def test_demo_corpus_tokenizer_has_26_characters():
    # docs/mesh-gpt.md:240-243
    with open(DEMO, encoding="utf-8") as f:
        t = G.CharacterTokenizer.from_text(f.read())
    assert t.vocab_size() == 26


# --------------------------------------------------------------- checkpoint

def _save(tmp_path, name, config, chars, params):
    path = str(tmp_path / name)
    G.Checkpoint(config, chars, params).save(path)
    return path, open(path, "rb").read()


def _read_bytes(tmp_path, data, name="probe.bin"):
    path = tmp_path / name
    path.write_bytes(data)
    return G.Checkpoint.load(str(path))


def test_checkpoint_round_trip_and_corruption(tmp_path):
    # checkpoint.rs:276-326
    chars = sorted("abcd ")
    config = G.GptConfig(vocab_size=5)
    params = G.initial_parameters(config, 7)
    path, data = _save(tmp_path, "m.bin", config, chars, params)
    assert data[:8] == b"MSHGPT07"
    assert struct.unpack("<7I", data[8:36]) == (5, 32, 32, 4, 2, 4, 6)
    assert struct.unpack("<5I", data[36:56]) == tuple(ord(c) for c in chars)
    assert len(data) == 56 + 4 * params.size
    loaded = G.Checkpoint.load(path)
    assert loaded.config == config
    assert loaded.characters == [ord(c) for c in chars]
    assert np.array_equal(loaded.parameters.view(np.uint32), params.view(np.uint32))
    for corrupted in (bytes(60), data[:-1], data + b"\0"):
        with pytest.raises(G.MeshGptError):
            _read_bytes(tmp_path, corrupted)
    with pytest.raises(G.MeshGptError, match="unexpected trailing checkpoint bytes"):
        _read_bytes(tmp_path, data + b"\0")
    for version, message in ((b"MSHGPT01", "retrain Mesh GPT with RoPE"), (b"MSHGPT02", "retrain Mesh GPT with RoPE"),
                             (b"MSHGPT03", "retrain Mesh GPT with RMSNorm"), (b"MSHGPT04", "retrain bias-free Mesh GPT"),
                             (b"MSHGPT05", "parameter-free QK-Norm"), (b"MSHGPT06", "mesh token embeddings"),
                             (b"MSHGPTXX", "unsupported Mesh GPT checkpoint format")):
        with pytest.raises(G.MeshGptError, match=message):
            _read_bytes(tmp_path, version + data[8:])
    nonfinite = data[:-4] + struct.pack("<f", float("nan"))
    with pytest.raises(G.MeshGptError, match="checkpoint parameters must contain only finite values"):
        _read_bytes(tmp_path, nonfinite)
    invalid = data[:8] + struct.pack("<I", 2**32 - 1) + data[12:]
    with pytest.raises(G.MeshGptError):
        _read_bytes(tmp_path, invalid)
    with pytest.raises(G.MeshGptError, match="cannot|No such|open"):
        G.Checkpoint.load(str(tmp_path / "missing.bin"))


def test_checkpoint_save_rejects_mismatch(tmp_path):
    # checkpoint.rs:26-31
    config = G.GptConfig(vocab_size=5)
    params = G.initial_parameters(config, 7)
    with pytest.raises(G.MeshGptError, match="checkpoint model, parameters, and tokenizer do not match"):
        G.Checkpoint(config, "abcd", params).save(str(tmp_path / "x.bin"))
    with pytest.raises(G.MeshGptError, match="checkpoint model, parameters, and tokenizer do not match"):
        G.Checkpoint(config, "abcde", params[1:]).save(str(tmp_path / "x.bin"))
    bad = params.copy()
    bad[0] = np.inf
    with pytest.raises(G.MeshGptError, match="checkpoint parameters must contain only finite values"):
        G.Checkpoint(config, "abcde", bad).save(str(tmp_path / "x.bin"))


def test_ablation_checkpoints_use_mshgpt08(tmp_path):
    # checkpoint.rs:328-378: field offsets 36 and 40 hold the embedding and connectivity codes.
    for embedding, connectivity in ((1, 0), (0, 1), (1, 1)):
        config = G.GptConfig(vocab_size=5, embedding=embedding, connectivity=connectivity)
        params = G.initial_parameters(config, 3)
        path, data = _save(tmp_path, f"a{embedding}{connectivity}.bin", config, "abcde", params)
        assert data[:8] == b"MSHGPT08"
        assert struct.unpack("<2I", data[36:44]) == (embedding, connectivity)
        loaded = G.Checkpoint.load(path)
        assert loaded.config == config
        assert np.array_equal(loaded.parameters, params)
        with pytest.raises(G.MeshGptError):
            _read_bytes(tmp_path, b"MSHGPT07" + data[8:])
        for field, message in ((36, "unknown checkpoint token embedding"), (40, "unknown checkpoint mesh connectivity")):
            unknown = data[:field] + struct.pack("<I", 2) + data[field + 4:]
            with pytest.raises(G.MeshGptError, match=message):
                _read_bytes(tmp_path, unknown)
        default = data[:36] + bytes(8) + data[44:]
        with pytest.raises(G.MeshGptError, match="the default architecture must use the MSHGPT07 layout"):
            _read_bytes(tmp_path, default)


def test_mshgpt09_layout_switches_and_geometry(tmp_path):
    # checkpoint.rs:61-78,146-168: a 09 file with default geometry and every
    # operator on must use an older layout; ablations round-trip through 09
    # with their fields at offsets 44..100; codes out of range are rejected.
    config = G.GptConfig(vocab_size=5)
    params = G.initial_parameters(config, 7)
    _, data = _save(tmp_path, "d.bin", config, "abcde", params)
    dims, rest = data[8:36], data[36:]
    # form, order, frequency, harmonics, overlap bits, normalization, frozen,
    # preserve, modulus, seed lo, seed hi -- defaults from src/gpt/geometry.rs:68-80
    geometry = [0, 0, 1, 1, 0, 0, 0, 0, 0, 0, 0]
    default09 = b"MSHGPT09" + dims + struct.pack("<2I", 0, 0) + struct.pack("<14I", *geometry, 1, 1, 1) + rest
    with pytest.raises(G.MeshGptError, match="default geometry must use an older checkpoint layout"):
        _read_bytes(tmp_path, default09)
    no_xsa = b"MSHGPT09" + dims + struct.pack("<2I", 0, 0) + struct.pack("<14I", *geometry, 1, 1, 0) + rest
    loaded = _read_bytes(tmp_path, no_xsa)
    assert loaded.config.xsa == 0 and loaded.config.rope == 1 and loaded.config.qk_norm == 1
    path, again = _save(tmp_path, "x.bin", loaded.config, "abcde", loaded.parameters)
    assert again == no_xsa
    for offset, code, message in ((100 - 12 + 8, 2, "invalid checkpoint switch"),
                                  (44, 10, "unknown checkpoint EmbeddingForm: 10"),
                                  (48, 3, "unknown checkpoint EmbeddingOrder: 3"),
                                  (64, 3, "unknown checkpoint EmbeddingNorm: 3"),
                                  (68, 2, "invalid checkpoint switch")):
        bad = no_xsa[:offset] + struct.pack("<I", code) + no_xsa[offset + 4:]
        with pytest.raises(G.MeshGptError, match=message):
            _read_bytes(tmp_path, bad)
    # A geometry ablation: circle codes in residue order of the mod-5 grok
    # vocabulary, a table embedding, protected coordinates; the writer picks 09.
    config = G.GptConfig(vocab_size=7, width=8, heads=2, embedding=1, form=1, order=1, modulus=5, seed=17,
                         preserve_features=2, qk_norm=0)
    params = G.initial_parameters(config, 3)
    path, data = _save(tmp_path, "g.bin", config, "abcdefg", params)
    assert data[:8] == b"MSHGPT09"
    assert struct.unpack("<16I", data[36:100]) == (1, 0, 1, 1, 1, 1, 0, 0, 0, 2, 5, 17, 0, 1, 0, 1)
    loaded = G.Checkpoint.load(path)
    assert loaded.config == config and np.array_equal(loaded.parameters, params)
    # Protected residual outputs must stay zero (config.rs:476-488), on save and load.
    offsets = O.group_offsets(O.config(**{k: v for k, v in config.as_dict().items() if k != "long_context"}))
    proj = offsets[1 + 3] + (config.attention_mesh_depth - 1) * 2 * config.width
    assert params[proj] == 0.0
    bad = params.copy()
    bad[proj] = 0.5
    with pytest.raises(G.MeshGptError, match="protected residual output weights must be zero"):
        G.Checkpoint(config, "abcdefg", bad).save(str(tmp_path / "bad.bin"))
    word = 100 + 7 * 4 + 4 * proj
    corrupt = data[:word] + struct.pack("<f", 0.5) + data[word + 4:]
    with pytest.raises(G.MeshGptError, match="protected residual output weights must be zero"):
        _read_bytes(tmp_path, corrupt)


# ---------------------------------------------------------------------- CLI

def _cli(*args):
    return subprocess.run([G.CLI_PATH, *args], capture_output=True, text=True, timeout=60)


def test_cli_help_and_argument_errors():
    r = _cli("--help")
    assert r.returncode == 0 and "--temperature" in r.stdout and "--checkpoint" in r.stdout
    r = _cli("generate", "--bogus")
    assert r.returncode == 1 and "unknown option: --bogus" in r.stderr
    r = _cli("generate", "--tokens", "-3")
    assert r.returncode == 1 and "invalid value for --tokens" in r.stderr
    r = _cli("generate", "--temperature", "-1")
    assert r.returncode == 1 and "temperature must be finite and nonnegative" in r.stderr
    r = _cli("verify")
    assert r.returncode == 1 and "run python tests/verify.py" in r.stderr
    r = _cli("train", "--dataset", "/nonexistent/corpus.txt")
    assert r.returncode == 1 and "cannot open dataset /nonexistent/corpus.txt" in r.stderr


def test_cli_init_writes_reference_checkpoint(tmp_path):
    # `init` seeds a checkpoint from a corpus: tokenizer from the text, weights
    # Layout::initialize(seed) (config.rs:416-459); the default architecture is MSHGPT07.
    path = str(tmp_path / "model.bin")
    r = _cli("init", "--dataset", DEMO, "--checkpoint", path, "--seed", "7")
    assert r.returncode == 0, r.stderr
    ck = G.Checkpoint.load(path)
    assert ck.config.vocab_size == 26 and ck.parameters.size == 3072
    o = O.config(vocab_size=26)
    assert np.array_equal(ck.parameters, O.initialize(o, 7))
    assert open(path, "rb").read(8) == b"MSHGPT07"
    r = _cli("init", "--dataset", DEMO, "--checkpoint", str(tmp_path / "b.bin"), "--connectivity", "butterfly",
             "--width", "64", "--embedding", "table")
    assert r.returncode == 0, r.stderr
    assert open(tmp_path / "b.bin", "rb").read(8) == b"MSHGPT08"
    r = _cli("init", "--dataset", DEMO, "--checkpoint", str(tmp_path / "c.bin"), "--connectivity", "Butterfly")
    assert r.returncode == 1
    # --init normal: N(0, 0.5^2) weights, the oracle's draw to the bit.
    r = _cli("init", "--dataset", DEMO, "--checkpoint", str(tmp_path / "n.bin"), "--init", "normal")
    assert r.returncode == 0, r.stderr
    ck = G.Checkpoint.load(str(tmp_path / "n.bin"))
    assert np.array_equal(ck.parameters, O.initialize_normal(o, 7, 0.5))
    r = _cli("init", "--dataset", DEMO, "--checkpoint", str(tmp_path / "s.bin"), "--init", "normal",
             "--init-sigma", "2", "--seed", "9")
    assert r.returncode == 0, r.stderr
    assert np.array_equal(G.Checkpoint.load(str(tmp_path / "s.bin")).parameters, O.initialize_normal(o, 9, 2.0))
    r = _cli("init", "--dataset", DEMO, "--checkpoint", str(tmp_path / "u.bin"), "--init", "uniform")
    assert r.returncode == 1 and "unknown initialisation: uniform; use reference or normal" in r.stderr
