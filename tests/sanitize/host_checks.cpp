// Host-side checks run under AddressSanitizer and UndefinedBehaviorSanitizer
// (tests/test_sanitizers.py builds and runs this file): the library's host
// types (configuration, layout, initialisation, token codes, geometry,
// tokenizer, checkpoint parsing of intact, truncated and corrupted files) and
// the CPU oracle's entry points, on small models.  Only memory safety and
// undefined behaviour are judged here; the values are checked elsewhere.
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "meshgpt_oracle.h"
#include "meshgpt_types.hpp"

using namespace meshgpt;

namespace {

int failures = 0;

void expect(bool ok, const char *what) {
    if (!ok) {
        std::fprintf(stderr, "check failed: %s\n", what);
        ++failures;
    }
}

template <class F>
bool throws(F &&f) {
    try {
        f();
    } catch (const Error &) {
        return true;
    }
    return false;
}

GptConfig small(size_t V = 11, size_t W = 16, size_t H = 2, size_t L = 2, size_t A = 3, size_t F = 4) {
    GptConfig c;
    c.vocab_size = V;
    c.context = 24;
    c.width = W;
    c.heads = H;
    c.layers = L;
    c.attention_mesh_depth = A;
    c.ffn_mesh_depth = F;
    return c;
}

std::vector<GptConfig> configs() {
    std::vector<GptConfig> out;
    out.push_back(GptConfig{});
    out.push_back(small());
    GptConfig t = small();
    t.embedding = TokenEmbedding::Table;
    out.push_back(t);
    GptConfig b = small(64, 128, 4, 2, 7, 7);
    b.connectivity = MeshConnectivity::Butterfly;
    out.push_back(b);
    GptConfig off = small();
    off.rope = off.qk_norm = off.xsa = false;
    out.push_back(off);
    const EmbeddingForm forms[] = {EmbeddingForm::Circle,    EmbeddingForm::Fourier,    EmbeddingForm::Orthogonal,
                                   EmbeddingForm::Simplex,   EmbeddingForm::Equiangular, EmbeddingForm::Antipodal,
                                   EmbeddingForm::Hypercube, EmbeddingForm::SignedPermutations,
                                   EmbeddingForm::Sphere};
    for (EmbeddingForm f : forms) {
        GptConfig g = small(11, 16);
        g.geometry.form = f;
        g.geometry.overlap = 0.25f;
        g.geometry.harmonics = 2;
        out.push_back(g);
    }
    GptConfig r = small(13, 32);
    r.geometry.form = EmbeddingForm::Circle;
    r.geometry.order = EmbeddingOrder::DiscreteLog;
    r.geometry.modulus = 11;
    r.geometry.seed = 7;
    out.push_back(r);
    GptConfig p = small(11, 16);
    p.geometry.form = EmbeddingForm::Orthogonal;
    p.geometry.preserve_features = 3;
    out.push_back(p);
    GptConfig n = small(11, 16);
    n.geometry.form = EmbeddingForm::Sphere;
    n.geometry.normalization = EmbeddingNorm::Rms;
    out.push_back(n);
    return out;
}

void host_types() {
    for (const GptConfig &c : configs()) {
        c.validate();
        const Layout layout = Layout::build(c);
        expect(layout.count() == c.parameter_count(), "layout count");
        for (uint64_t seed : {uint64_t(0), uint64_t(7), std::numeric_limits<uint64_t>::max()}) {
            const std::vector<float> p = layout.initialize(c, seed);
            expect(p.size() == c.parameter_count(), "parameter count");
            layout.validate_constraints(c, p.data());
            if (seed == 7 && c.embedding == TokenEmbedding::Mesh) {
                GptConfig table = c;
                table.embedding = TokenEmbedding::Table;
                expect(tabulate_embedding(c, p).size() == table.parameter_count(), "tabulated parameter count");
            }
        }
        const std::vector<float> codes = token_codes(c);
        expect(codes.size() == c.vocab_size * c.width, "token codes size");
        std::vector<uint32_t> tokens(12);
        for (size_t i = 0; i < tokens.size(); ++i) tokens[i] = uint32_t(i % c.vocab_size);
        c.validate_tokens(tokens.data(), tokens.size(), 6);
        tokens[3] = uint32_t(c.vocab_size);
        expect(throws([&] { c.validate_tokens(tokens.data(), tokens.size(), 6); }), "token out of range");
    }
    // Invalid configurations throw the reference's errors.
    GptConfig bad = small();
    bad.width = 15;
    expect(throws([&] { bad.validate(); }), "width not divisible by heads");
    bad = small();
    bad.vocab_size = 0;
    expect(throws([&] { bad.validate(); }), "empty vocabulary");
    bad = small(11, 8);
    bad.geometry.form = EmbeddingForm::Orthogonal;
    expect(throws([&] { bad.validate(); }), "orthogonal codes need width >= vocabulary");
    bad = small();
    bad.geometry.order = EmbeddingOrder::Residue;
    bad.geometry.modulus = 12;
    expect(throws([&] { bad.validate(); }), "residue order needs a prime");

    const std::vector<uint32_t> perm = residue_permutation(97, 7);
    std::vector<int> seen(97, 0);
    for (uint32_t t : perm) seen[t] += 1;
    for (int k : seen) expect(k == 1, "residue permutation");
    expect(primitive_root(97) == 5, "primitive root of 97");

    Random rng(7);
    for (int i = 0; i < 1000; ++i) {
        expect(rng.index(13) < 13, "Random::index bound");
        const float u = rng.unit();
        expect(u >= 0.0f && u < 1.0f, "Random::unit range");
    }

    const CharacterTokenizer tok = CharacterTokenizer::from_text("hello, wörld\n");
    const std::vector<uint32_t> ids = tok.encode("wörld, hello");
    expect(tok.decode(ids.data(), ids.size()) == "wörld, hello", "tokenizer round trip");
    expect(throws([&] { tok.encode("xyz"); }), "unknown character");
    expect(throws([&] { tok.encode(std::string("\xff\xfe")); }), "invalid UTF-8");
    const uint32_t out_of_range = uint32_t(tok.vocab_size());
    expect(throws([&] { tok.decode(&out_of_range, 1); }), "token past the vocabulary");
}

void checkpoints() {
    for (const GptConfig &c : configs()) {
        if (c.vocab_size > 64) continue;
        Checkpoint ck;
        ck.config = c;
        std::vector<uint32_t> chars;
        for (size_t i = 0; i < c.vocab_size; ++i) chars.push_back(uint32_t('A' + i));
        ck.tokenizer = CharacterTokenizer::from_characters(chars);
        ck.parameters = Layout::build(c).initialize(c, 3);
        const std::vector<uint8_t> bytes = ck.serialize();
        const Checkpoint back = Checkpoint::read(bytes.data(), bytes.size());
        expect(back.config == c && back.tokenizer == ck.tokenizer && back.parameters == ck.parameters,
               "checkpoint round trip");
        // Every truncation is rejected; the file's header bytes, corrupted one
        // at a time, are parsed or rejected without touching memory outside
        // the buffer.
        for (size_t n = 0; n < bytes.size(); n += (n < 256 ? 1 : 97))
            expect(throws([&] { Checkpoint::read(bytes.data(), n); }), "truncated checkpoint");
        for (size_t i = 0; i < std::min<size_t>(bytes.size(), 160); ++i) {
            std::vector<uint8_t> bad = bytes;
            bad[i] ^= 0xA5;
            try {
                (void)Checkpoint::read(bad.data(), bad.size());
            } catch (const Error &) {
            }
        }
        std::vector<uint8_t> longer = bytes;
        longer.push_back(0);
        expect(throws([&] { Checkpoint::read(longer.data(), longer.size()); }), "trailing bytes");
    }
}

og_config to_og(const GptConfig &c) {
    og_config o{};
    o.vocab_size = uint32_t(c.vocab_size);
    o.context = uint32_t(c.context);
    o.width = uint32_t(c.width);
    o.heads = uint32_t(c.heads);
    o.layers = uint32_t(c.layers);
    o.attention_mesh_depth = uint32_t(c.attention_mesh_depth);
    o.ffn_mesh_depth = uint32_t(c.ffn_mesh_depth);
    o.embedding = uint32_t(c.embedding);
    o.connectivity = uint32_t(c.connectivity);
    o.rope = c.rope;
    o.qk_norm = c.qk_norm;
    o.xsa = c.xsa;
    o.form = uint32_t(c.geometry.form);
    o.order = uint32_t(c.geometry.order);
    o.frequency = uint32_t(c.geometry.frequency);
    o.harmonics = uint32_t(c.geometry.harmonics);
    o.overlap = c.geometry.overlap;
    o.normalization = uint32_t(c.geometry.normalization);
    o.frozen = c.geometry.frozen;
    o.preserve_features = uint32_t(c.geometry.preserve_features);
    o.modulus = uint32_t(c.geometry.modulus);
    o.seed = c.geometry.seed;
    return o;
}

void oracle() {
    for (const GptConfig &c : configs()) {
        if (c.width > 32) continue;
        const og_config o = to_og(c);
        char err[256];
        expect(og_validate(&o, 0, err, sizeof err) == 0, "oracle validation");
        const size_t n = og_parameter_count(&o), V = c.vocab_size, W = c.width;
        std::vector<float> params(n);
        og_initialize(&o, 7, params.data());
        std::vector<double> emb(V * W), logits(12 * V), hidden(12 * W);
        expect(og_token_embeddings(&o, params.data(), emb.data()) == 0, "oracle embeddings");
        std::vector<uint32_t> tokens(12);
        for (size_t i = 0; i < tokens.size(); ++i) tokens[i] = uint32_t((5 * i + 1) % V);
        expect(og_logits(&o, params.data(), tokens.data(), 12, 6, logits.data()) == 0, "oracle logits");
        expect(og_hidden_states(&o, params.data(), tokens.data(), 12, 6, hidden.data()) == 0, "oracle hidden");
        std::vector<uint32_t> targets(tokens.begin() + 1, tokens.end());
        targets.push_back(UINT32_MAX);
        double loss = 0.0;
        expect(og_cross_entropy(&o, params.data(), tokens.data(), targets.data(), 12, 6, &loss) == 0,
               "oracle cross-entropy");
        // Generation past the context slides the window; the cached loop
        // stops at the context.
        const uint32_t prompt[3] = {1, 2, 3};
        std::vector<uint32_t> out(3 + 30), cached(3 + 20);
        std::vector<float> last(V);
        expect(og_generate(&o, params.data(), prompt, 3, 30, 0.7f, 5, out.data()) == 0, "oracle generate");
        expect(og_generate_cached(&o, params.data(), prompt, 3, 20, 0.0f, 5, cached.data(), last.data()) == 0,
               "oracle cached generate");
        std::vector<float> row(V);
        for (size_t t = 0; t < V; ++t) row[t] = float(logits[t]);
        uint64_t state = 9;
        expect(og_sample(row.data(), V, 0.9f, &state) < V, "oracle sample");
        size_t pred = 0;
        (void)og_row_metrics(row.data(), V, 0, &pred);
    }
    std::vector<uint32_t> residues(97), train(3 * 9409), valid(3 * 9409);
    size_t nt = 0, nv = 0;
    expect(og_equations(97, 0, 0.5, 7, residues.data(), train.data(), valid.data(), &nt, &nv) >= 0 &&
               nt + nv == 9409,
           "oracle equations");
    std::vector<uint32_t> corpus(500), inputs(4 * 16), tgt(4 * 16);
    for (size_t i = 0; i < corpus.size(); ++i) corpus[i] = uint32_t(i * 7 % 31);
    expect(og_text_batch(corpus.data(), corpus.size(), 0, 16, 4, 3, inputs.data(), tgt.data()) == 0,
           "oracle text batch");
}

}  // namespace

int main() {
    try {
        host_types();
        checkpoints();
        oracle();
    } catch (const std::exception &e) {
        std::fprintf(stderr, "unexpected exception: %s\n", e.what());
        return 2;
    }
    if (failures) return 1;
    std::printf("host checks ok\n");
    return 0;
}
