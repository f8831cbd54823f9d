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
                               ffn_mesh_depth=6, embedding=0, connectivity=0, long_context=0)
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


def test_mshgpt09_default_geometry_rejected_and_ablations_unsupported(tmp_path):
    # checkpoint.rs:146-168: a 09 file with default geometry and every operator
    # on must use an older layout; one that changes them is a geometry ablation
    # this build does not run (status MG_UNSUPPORTED).
    config = G.GptConfig(vocab_size=5)
    params = G.initial_parameters(config, 7)
    _, data = _save(tmp_path, "d.bin", config, "abcde", params)
    dims, rest = data[8:36], data[36:]
    # form, order, frequency, harmonics, overlap bits, normalization, frozen,
    # preserve, modulus, seed lo, seed hi, rope, qk_norm, xsa -- defaults from
    # src/gpt/geometry.rs:68-80 (Parity, Token, 1, 1, 0.0, None, false, 0, 0, 0)
    geometry = [0, 0, 1, 1, 0, 0, 0, 0, 0, 0, 0]
    default09 = b"MSHGPT09" + dims + struct.pack("<2I", 0, 0) + struct.pack("<14I", *geometry, 1, 1, 1) + rest
    with pytest.raises(G.MeshGptError, match="default geometry must use an older checkpoint layout"):
        _read_bytes(tmp_path, default09)
    no_xsa = b"MSHGPT09" + dims + struct.pack("<2I", 0, 0) + struct.pack("<14I", *geometry, 1, 1, 0) + rest
    with pytest.raises(G.MeshGptError) as info:
        _read_bytes(tmp_path, no_xsa)
    assert info.value.status == G.MG_UNSUPPORTED
    bad_switch = b"MSHGPT09" + dims + struct.pack("<2I", 0, 0) + struct.pack("<14I", *geometry, 1, 1, 2) + rest
    with pytest.raises(G.MeshGptError, match="invalid checkpoint switch"):
        _read_bytes(tmp_path, bad_switch)


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
    r = _cli("train")
    assert r.returncode == 1 and "not part of this build" in r.stderr


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
