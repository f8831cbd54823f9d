// Token-code geometry of the MSHGPT09 ablations (src/gpt/geometry.rs): the
// constraints on a configuration, the token order of arithmetic vocabularies
// and the geometric code families.  Compiled without floating-point
// contraction, like the rest of the host types: every code value is computed
// in f64 and rounded to f32 exactly as the reference does.
#include <charconv>
#include <cmath>

#include "meshgpt_types.hpp"

namespace meshgpt {

namespace {

size_t bit_length(size_t x) {
    size_t n = 0;
    for (; x; x >>= 1) ++n;
    return n;
}

bool is_prime(size_t n) {
    if (n < 2) return false;
    for (size_t d = 2; d < n; ++d)
        if (n % d == 0) return false;
    return true;
}

// The token at each position of the geometric order, and the length of the
// cyclic part (geometry.rs:186-211).
std::pair<std::vector<size_t>, size_t> ordered_tokens(const GptConfig &config) {
    const EmbeddingGeometry &g = config.geometry;
    std::vector<size_t> order;
    if (g.order == EmbeddingOrder::Token) {
        for (size_t t = 0; t < config.vocab_size; ++t) order.push_back(t);
        return {order, config.vocab_size};
    }
    const std::vector<uint32_t> ids = residue_permutation(g.modulus, g.seed);
    if (g.order == EmbeddingOrder::Residue) {
        for (uint32_t id : ids) order.push_back(id);
    } else {
        const size_t root = primitive_root(g.modulus);
        size_t residue = 1;
        for (size_t k = 0; k + 1 < g.modulus; ++k) {
            order.push_back(ids[residue]);
            residue = residue * root % g.modulus;
        }
    }
    const size_t cycle = order.size();
    if (g.order == EmbeddingOrder::DiscreteLog) order.push_back(ids[0]);
    order.push_back(g.modulus);
    order.push_back(g.modulus + 1);
    return {order, cycle};
}

// Helmert coordinates of a regular unit simplex in R^(n-1) (geometry.rs:226-236).
double simplex_coordinate(size_t row, size_t column, size_t n) {
    const double scale = std::sqrt(double(n) / double(n - 1));
    const double denominator = std::sqrt(double((column + 1) * (column + 2)));
    if (row <= column) return scale / denominator;
    if (row == column + 1) return -scale * double(column + 1) / denominator;
    return 0.0;
}

constexpr double kTau = 6.283185307179586;

}  // namespace

bool EmbeddingGeometry::operator==(const EmbeddingGeometry &o) const {
    return form == o.form && order == o.order && frequency == o.frequency && harmonics == o.harmonics &&
           (overlap == o.overlap || (std::isnan(overlap) && std::isnan(o.overlap))) &&
           normalization == o.normalization && frozen == o.frozen && preserve_features == o.preserve_features &&
           modulus == o.modulus && seed == o.seed;
}

float EmbeddingGeometry::radius(size_t width) const {
    return normalization == EmbeddingNorm::Rms ? std::sqrt(float(width)) : 1.0f;
}

void EmbeddingGeometry::validate(const GptConfig &config) const {
    const size_t v = config.vocab_size, w = config.width;
    if (frequency == 0 || frequency > 0xFFFFFFFFull || harmonics == 0 || harmonics > w / 2)
        throw Error("embedding frequency must be positive and harmonics in 1..width/2");
    if (!std::isfinite(overlap) || preserve_features > w)
        throw Error("embedding overlap must be finite; preserved features must fit width");
    if (modulus > 0xFFFFFFFFull) throw Error("embedding modulus exceeds checkpoint field capacity");
    if (preserve_features > 0 && normalization != EmbeddingNorm::None)
        throw Error("preserved coordinates require --embedding-norm none; full-vector normalization would "
                    "rescale the protected feature");
    bool fits = true;
    switch (form) {
    case EmbeddingForm::Orthogonal: fits = w >= v; break;
    case EmbeddingForm::Simplex: fits = w + 1 >= v; break;
    case EmbeddingForm::Equiangular: {
        const float lower = -1.0f / float(v - 1);
        fits = overlap >= lower && overlap <= 1.0f && (overlap == 1.0f || w + (overlap == lower ? 1 : 0) >= v);
        break;
    }
    case EmbeddingForm::Hypercube: fits = w >= bit_length(v - 1); break;
    case EmbeddingForm::SignedPermutations: fits = w >= 4 && v <= 256; break;
    default: break;
    }
    if (!fits)
        throw Error(std::string(name(form)) + " embedding does not fit vocabulary " + std::to_string(v) +
                    ", width " + std::to_string(w) + ", overlap " + display_f32(overlap));
    if (order != EmbeddingOrder::Token) {
        if (modulus < 2 || modulus > 254 || !is_prime(modulus) || v != modulus + 2)
            throw Error("arithmetic embedding order requires a grok prime and vocabulary modulus+2");
        // Independent directions for zero (discrete-log), the operation and '='.
        const size_t special = 2 + (order == EmbeddingOrder::DiscreteLog ? 1 : 0);
        const size_t pairs = form == EmbeddingForm::Fourier ? harmonics : 1;
        if ((form == EmbeddingForm::Circle || form == EmbeddingForm::Fourier) && w < 2 * pairs + special)
            throw Error("arithmetic circle/Fourier codes need extra coordinates for special symbols");
    }
}

std::vector<uint32_t> residue_permutation(size_t modulus, uint64_t seed) {
    std::vector<uint32_t> tokens(modulus);
    for (size_t i = 0; i < modulus; ++i) tokens[i] = uint32_t(i);
    Random symbols(seed ^ 0x73796d626f6c7301ULL);
    for (size_t end = modulus; end-- > 1;) std::swap(tokens[end], tokens[symbols.index(end + 1)]);
    return tokens;
}

namespace {

uint64_t modular_inverse(uint64_t value, uint64_t modulus) {  // grokking.rs:94-106 (Fermat)
    uint64_t result = 1, base = value % modulus;
    for (uint64_t e = modulus - 2; e; e >>= 1) {
        if (e & 1) result = result * base % modulus;
        base = base * base % modulus;
    }
    return result;
}

// ModularOperation::apply (grokking.rs:52-67), codes in declaration order.
size_t apply_operation(uint32_t op, uint64_t a, uint64_t b, uint64_t p) {
    switch (op) {
    case 0: return (a + b) % p;
    case 1: return a * b % p;
    case 2: return (a + p - b) % p;
    case 3: return a * modular_inverse(b, p) % p;
    case 4: return b % 2 == 1 ? a * modular_inverse(b, p) % p : (a + p - b) % p;
    case 5: return (a * a + b * b) % p;
    case 6: return (a * a + a * b + b * b) % p;
    case 7: return (a * a + a * b + b * b + a) % p;
    case 8: return (a * a * a + a * b) % p;
    default: return (a * a * a + a * b * b + b) % p;
    }
}

}  // namespace

EquationDataset EquationDataset::build(size_t modulus, uint32_t operation, double train_fraction, uint64_t seed) {
    bool prime = modulus >= 2 && modulus <= 254;  // MAX_VOCAB (256, src/gpt/mod.rs:29) - 2
    for (size_t d = 2; prime && d < modulus; ++d) prime = modulus % d != 0;
    if (!prime) throw Error("modulus must be a prime in 2..254 (two vocabulary slots are reserved)");
    if (operation > 9) throw Error("unknown modular operation");
    if (!std::isfinite(train_fraction) || !(train_fraction > 0.0 && train_fraction < 1.0))
        throw Error("train fraction must be finite and strictly between 0 and 1");
    EquationDataset d;
    d.modulus = modulus;
    d.operation = operation;
    d.residue_tokens = residue_permutation(modulus, seed);
    std::vector<Equation> all;
    for (size_t a = 0; a < modulus; ++a)
        for (size_t b = operation == 3 ? 1 : 0; b < modulus; ++b)
            all.push_back({a, b, apply_operation(operation, a, b, modulus)});
    const size_t split = size_t(std::floor(double(all.size()) * train_fraction));
    if (split < 2 || split >= all.size())
        throw Error("split needs at least two training equations and one validation equation");
    Random splits(seed ^ 0x73706c6974730002ULL);
    for (size_t end = all.size(); end-- > 1;) std::swap(all[end], all[splits.index(end + 1)]);
    d.training.assign(all.begin(), all.begin() + split);
    d.validation.assign(all.begin() + split, all.end());
    return d;
}

void EquationDataset::batch(bool validation, const size_t *indices, size_t n, uint32_t *inputs,
                            uint32_t *targets) const {
    if (n == 0 || n > kMaxRows / 4) throw Error("equation batches need 1..32768 examples");
    const std::vector<Equation> &split = validation ? this->validation : training;
    for (size_t i = 0; i < n; ++i) {
        if (indices[i] >= split.size()) throw Error("equation index is outside the split");
        const Equation &e = split[indices[i]];
        const uint32_t row[4] = {residue_tokens[e.a], uint32_t(modulus), residue_tokens[e.b], uint32_t(modulus + 1)};
        const uint32_t want[4] = {kIgnoreTarget, kIgnoreTarget, kIgnoreTarget, residue_tokens[e.answer]};
        std::copy(row, row + 4, inputs + 4 * i);
        std::copy(want, want + 4, targets + 4 * i);
    }
}

CharacterTokenizer EquationDataset::tokenizer() const {
    std::vector<uint32_t> characters(modulus + 2, uint32_t(' '));
    for (size_t r = 0; r < residue_tokens.size(); ++r) characters[residue_tokens[r]] = 0xE000u + uint32_t(r);
    static const uint32_t symbols[] = {'+', '*', '-', '/'};  // ModularOperation::symbol
    characters[modulus] = operation < 4 ? symbols[operation] : 0x2218u;
    characters[modulus + 1] = uint32_t('=');
    return CharacterTokenizer::from_characters(characters);
}

size_t primitive_root(size_t prime) {
    if (prime == 2) return 1;
    for (size_t g = 2; g < prime; ++g) {
        std::vector<bool> seen(prime, false);
        size_t x = 1;
        bool ok = true;
        for (size_t k = 0; k + 1 < prime; ++k) {
            if (seen[x]) {
                ok = false;
                break;
            }
            seen[x] = true;
            x = x * g % prime;
        }
        if (ok && x == 1) return g;
    }
    throw Error("a prime has a primitive root");
}

// Parity codes, computed for positions 0..V-1, belong to the tokens of the
// geometric order (geometry.rs:213-222).
std::vector<float> reorder_parity(const GptConfig &config, const std::vector<float> &codes) {
    if (config.geometry.order == EmbeddingOrder::Token) return codes;
    const size_t W = config.width;
    const std::vector<size_t> order = ordered_tokens(config).first;
    std::vector<float> result(codes.size());
    for (size_t i = 0; i < order.size(); ++i)
        std::copy(codes.begin() + i * W, codes.begin() + (i + 1) * W, result.begin() + order[i] * W);
    return result;
}

// geometry.rs:238-325: the geometric code of each token, V x W.
std::vector<float> geometric_codes(const GptConfig &config) {
    const size_t v = config.vocab_size, w = config.width;
    const EmbeddingGeometry &g = config.geometry;
    const auto [order, cycle] = ordered_tokens(config);
    std::vector<float> codes(v * w, 0.0f);
    Random random(g.seed ^ 0x5350484552453031ULL);
    for (size_t row = 0; row < order.size(); ++row) {
        float *code = codes.data() + order[row] * w;
        switch (g.form) {
        case EmbeddingForm::Parity: throw Error("parity codes use the original generator");
        case EmbeddingForm::Circle:
        case EmbeddingForm::Fourier: {
            const size_t pairs = g.form == EmbeddingForm::Fourier ? g.harmonics : 1;
            if (row >= cycle) {
                code[2 * pairs + row - cycle] = 1.0f;
            } else {
                const double scale = 1.0 / std::sqrt(double(pairs));
                for (size_t pair = 0; pair < pairs; ++pair) {
                    const size_t frequency = (g.frequency % cycle + pair % cycle) % cycle;
                    const double angle = kTau * double(frequency) * double(row) / double(cycle);
                    code[2 * pair] = float(scale * std::cos(angle));
                    code[2 * pair + 1] = float(scale * std::sin(angle));
                }
            }
            break;
        }
        case EmbeddingForm::Orthogonal: code[row] = 1.0f; break;
        case EmbeddingForm::Simplex:
        case EmbeddingForm::Equiangular: {
            const double rho = g.form == EmbeddingForm::Simplex ? -1.0 / double(v - 1) : double(g.overlap);
            if (rho == 1.0) {
                code[0] = 1.0f;
                break;
            }
            const double a = std::sqrt((1.0 - rho) * double(v - 1) / double(v));
            for (size_t c = 0; c + 1 < v; ++c) code[c] = float(a * simplex_coordinate(row, c, v));
            if (w >= v) code[v - 1] = float(std::sqrt(std::max(1.0 + double(v - 1) * rho, 0.0) / double(v)));
            break;
        }
        case EmbeddingForm::Antipodal: code[0] = row % 2 == 0 ? 1.0f : -1.0f; break;
        case EmbeddingForm::Hypercube: {
            const size_t bits = bit_length(v - 1);
            for (size_t bit = 0; bit < bits; ++bit)
                code[bit] = ((row & (size_t(1) << bit)) == 0 ? -1.0f : 1.0f) / std::sqrt(float(bits));
            break;
        }
        case EmbeddingForm::SignedPermutations: {
            const size_t p = row / 16;
            for (size_t c = 0; c < 4; ++c) {
                const size_t slot = c < 2 ? (c + p / 2 % 2) % 2 : 2 + (c - 2 + p % 2) % 2;
                const float magnitude = float(1 + (slot + p / 4) % 4);
                code[c] = magnitude * ((row & (size_t(1) << c)) == 0 ? 1.0f : -1.0f);
            }
            break;
        }
        case EmbeddingForm::Sphere: {
            double squares = 0.0;
            for (size_t c = 0; c < w; ++c) {
                const double radius = std::sqrt(-2.0 * std::log(double(std::max(random.unit(), 1.0f / 16777216.0f))));
                const double angle = kTau * double(random.unit());
                code[c] = float(radius * std::cos(angle));
                squares += double(code[c]) * double(code[c]);
            }
            for (size_t c = 0; c < w; ++c) code[c] = float(double(code[c]) / std::sqrt(squares));
            break;
        }
        }
    }
    return codes;
}

}  // namespace meshgpt
