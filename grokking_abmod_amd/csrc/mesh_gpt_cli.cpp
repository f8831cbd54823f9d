// mesh-gpt: the reference's `mesh-gpt generate` and `mesh-gpt train` commands
// (src/bin/mesh-gpt.rs:29-299, the geometry flags of src/bin/mesh-gpt/
// geometry.rs:5-55) on the MI355X library, with the same flags, defaults,
// output, artifacts and error text.  Extensions: --batch N for generate (N
// sequences, seeds seed..seed+N-1, one line each), --config NAME with
// --random-prompt LEN (a seeded synthetic model and prompt, no checkpoint), and
// `init` (write a seeded checkpoint).
#include <charconv>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "meshgpt_types.hpp"
#include "model.hpp"

using namespace meshgpt;

namespace {

struct Options {
    std::string command = "train";
    GptConfig config;
    GptTrainOptions training;
    size_t device = 0;
    uint64_t seed = 7;
    size_t batch = 1;
    bool batch_set = false;
    std::string dataset = "data/mesh-gpt-demo.txt";
    std::string output = "target/mesh-gpt";
    std::string checkpoint;
    std::string prompt = "the little robot ";
    size_t tokens = 240;
    float temperature = 0.7f;
    std::string synthetic;
    size_t random_prompt = 0;
    std::string prompt_file;
    std::string init = "reference";
    float init_sigma = 0.5f;
    bool help = false;
};

// cli::value (src/cli.rs:7-13)
template <class T>
T value(std::vector<std::string>::const_iterator &it, std::vector<std::string>::const_iterator end,
        const std::string &flag) {
    if (++it == end) throw Error("missing value for " + flag);
    const std::string &text = *it;
    try {
        size_t used = 0;
        if constexpr (std::is_same_v<T, float>) {
            float v = std::stof(text, &used);
            if (used != text.size()) throw 0;
            return v;
        } else if constexpr (std::is_same_v<T, double>) {
            double v = std::stod(text, &used);
            if (used != text.size()) throw 0;
            return v;
        } else if constexpr (std::is_same_v<T, std::string>) {
            return text;
        } else {
            if (text.empty() || text[0] == '-' || text[0] == '+') throw 0;
            unsigned long long v = std::stoull(text, &used, 10);
            if (used != text.size()) throw 0;
            return T(v);
        }
    } catch (...) {
        throw Error("invalid value for " + flag + ": " + text);
    }
}

GptConfig named_config(const std::string &name) {
    // Synthetic workloads of the benchmark (vocabulary, width, heads, layers,
    // depths, context); all butterfly meshes except the symbolic one.
    GptConfig c;
    c.connectivity = MeshConnectivity::Butterfly;
    if (name == "tiny") {
        c.vocab_size = 64, c.width = 128, c.heads = 4, c.layers = 2, c.attention_mesh_depth = 7,
        c.ffn_mesh_depth = 7, c.context = 256;
    } else if (name == "mid") {
        c.vocab_size = 256, c.width = 512, c.heads = 8, c.layers = 6, c.attention_mesh_depth = 9,
        c.ffn_mesh_depth = 9, c.context = 1024;
    } else if (name == "long") {
        c.vocab_size = 256, c.width = 512, c.heads = 8, c.layers = 4, c.attention_mesh_depth = 9,
        c.ffn_mesh_depth = 9, c.context = 8448, c.long_context = true;
    } else if (name == "high") {
        c.vocab_size = 256, c.width = 1024, c.heads = 16, c.layers = 12, c.attention_mesh_depth = 10,
        c.ffn_mesh_depth = 10, c.context = 2048;
    } else if (name == "symbolic") {
        c = GptConfig{};
        c.vocab_size = 99, c.width = 128, c.context = 4;
    } else {
        throw Error("unknown config: " + name + "; use tiny, symbolic, mid, long or high");
    }
    return c;
}

// "--rope 0|1" and the like (geometry.rs:50-55).
bool switch_value(std::vector<std::string>::const_iterator &it, std::vector<std::string>::const_iterator end,
                  const std::string &flag) {
    const uint32_t v = value<uint32_t>(it, end, flag);
    if (v > 1) throw Error(flag + " requires 0 or 1");
    return v == 1;
}

// A named value (cli::value over FromStr): a name the parser refuses is
// "invalid value for FLAG: TEXT".
template <class F>
auto named(std::vector<std::string>::const_iterator &it, std::vector<std::string>::const_iterator end,
           const std::string &flag, F &&parse) {
    const std::string text = value<std::string>(it, end, flag);
    try {
        return parse(text);
    } catch (const Error &) {
        throw Error("invalid value for " + flag + ": " + text);
    }
}

// The shared geometry flags (geometry.rs:24-48); false for any other flag.
bool geometry_option(GptConfig &c, const std::string &flag, std::vector<std::string>::const_iterator &it,
                     std::vector<std::string>::const_iterator end) {
    EmbeddingGeometry &g = c.geometry;
    if (flag == "--embedding") c.embedding = named(it, end, flag, parse_embedding);
    else if (flag == "--connectivity") c.connectivity = named(it, end, flag, parse_connectivity);
    else if (flag == "--embedding-form") g.form = named(it, end, flag, parse_form);
    else if (flag == "--embedding-order") g.order = named(it, end, flag, parse_order);
    else if (flag == "--embedding-frequency") g.frequency = value<size_t>(it, end, flag);
    else if (flag == "--embedding-harmonics") g.harmonics = value<size_t>(it, end, flag);
    else if (flag == "--equiangular-overlap") g.overlap = value<float>(it, end, flag);
    else if (flag == "--embedding-norm") g.normalization = named(it, end, flag, parse_norm);
    else if (flag == "--freeze-embedding") g.frozen = true;
    else if (flag == "--preserve-features") g.preserve_features = value<size_t>(it, end, flag);
    else if (flag == "--geometry-seed") g.seed = value<uint64_t>(it, end, flag);
    else if (flag == "--rope") c.rope = switch_value(it, end, flag);
    else if (flag == "--qk-norm") c.qk_norm = switch_value(it, end, flag);
    else if (flag == "--xsa") c.xsa = switch_value(it, end, flag);
    else return false;
    return true;
}

// geometry::metadata (geometry.rs:56-75): the run's geometry.txt.
std::string geometry_metadata(const GptConfig &c) {
    const EmbeddingGeometry &g = c.geometry;
    auto b = [](bool v) { return v ? "true" : "false"; };
    std::string s;
    s += "embedding_form=" + std::string(name(g.form)) + "\n";
    s += "embedding_order=" + std::string(name(g.order)) + "\n";
    s += "embedding_frequency=" + std::to_string(g.frequency) + "\n";
    s += "embedding_harmonics=" + std::to_string(g.harmonics) + "\n";
    s += "equiangular_overlap=" + display_f32(g.overlap) + "\n";
    s += "embedding_norm=" + std::string(name(g.normalization)) + "\n";
    s += "freeze_embedding=" + std::string(b(g.frozen)) + "\n";
    s += "preserve_features=" + std::to_string(g.preserve_features) + "\n";
    s += "geometry_modulus=" + std::to_string(g.modulus) + "\n";
    s += "geometry_seed=" + std::to_string(g.seed) + "\n";
    s += "rope=" + std::string(b(c.rope)) + "\n";
    s += "qk_norm_enabled=" + std::string(b(c.qk_norm)) + "\n";
    s += "xsa_enabled=" + std::string(b(c.xsa)) + "\n";
    s += "geometry_supplies_arithmetic_order=" + std::string(b(g.order != EmbeddingOrder::Token)) + "\n";
    return s;
}

std::string format(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
std::string format(const char *fmt, ...) {
    char buf[512];
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, args);
    va_end(args);
    return buf;
}

std::string read_file(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error("cannot open dataset " + path, kIo);
    return std::string(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

void write_file(const std::filesystem::path &path, const std::string &text) {
    std::ofstream f(path, std::ios::binary);
    if (!(f << text)) throw Error("cannot write " + path.string(), kIo);
}

Options parse(int argc, char **argv) {
    std::vector<std::string> args(argv + 1, argv + argc);
    Options o;
    auto it = args.cbegin();
    if (it != args.cend() && !it->empty() && (*it)[0] != '-') o.command = *it++;
    for (; it != args.cend(); ++it) {
        const std::string flag = *it;
        auto end = args.cend();
        if (flag == "--width") o.config.width = value<size_t>(it, end, flag);
        else if (flag == "--heads") o.config.heads = value<size_t>(it, end, flag);
        else if (flag == "--layers") o.config.layers = value<size_t>(it, end, flag);
        else if (flag == "--context") o.config.context = value<size_t>(it, end, flag);
        else if (flag == "--attention-depth") o.config.attention_mesh_depth = value<size_t>(it, end, flag);
        else if (flag == "--ffn-depth") o.config.ffn_mesh_depth = value<size_t>(it, end, flag);
        else if (flag == "--steps") o.training.steps = value<size_t>(it, end, flag);
        else if (flag == "--learning-rate") o.training.learning_rate = value<float>(it, end, flag);
        else if (flag == "--weight-decay") o.training.weight_decay = value<float>(it, end, flag);
        else if (flag == "--report-every") o.training.report_every = value<size_t>(it, end, flag);
        else if (geometry_option(o.config, flag, it, end)) continue;
        else if (flag == "--batch") o.batch = value<size_t>(it, end, flag), o.batch_set = true;
        else if (flag == "--seed") o.seed = value<uint64_t>(it, end, flag);
        else if (flag == "--device") o.device = value<size_t>(it, end, flag);
        else if (flag == "--dataset") o.dataset = value<std::string>(it, end, flag);
        else if (flag == "--output") o.output = value<std::string>(it, end, flag);
        else if (flag == "--checkpoint") o.checkpoint = value<std::string>(it, end, flag);
        else if (flag == "--prompt") o.prompt = value<std::string>(it, end, flag);
        else if (flag == "--tokens") o.tokens = value<size_t>(it, end, flag);
        else if (flag == "--temperature") o.temperature = value<float>(it, end, flag);
        else if (flag == "--config") o.synthetic = value<std::string>(it, end, flag);
        else if (flag == "--random-prompt") o.random_prompt = value<size_t>(it, end, flag);
        else if (flag == "--prompt-file") o.prompt_file = value<std::string>(it, end, flag);
        else if (flag == "--init") o.init = value<std::string>(it, end, flag);
        else if (flag == "--init-sigma") o.init_sigma = value<float>(it, end, flag);
        else if (flag == "--help" || flag == "-h") o.help = true;
        else throw Error("unknown option: " + flag + "; use --help");
    }
    return o;
}

// geometry::HELP (geometry.rs:5-22)
const char *kGeometryHelp =
    "--embedding mesh|table  Tied embedding parameterization (default: mesh)\n"
    "--connectivity neighbor|butterfly  Mesh parents (default: neighbor)\n"
    "--embedding-form NAME  parity (default), circle, fourier, orthogonal, simplex,\n"
    "                       equiangular, antipodal, hypercube, signed-permutations, sphere\n"
    "--embedding-order NAME token (default), residue, discrete-log; arithmetic order is grok-only\n"
    "--embedding-frequency N  First cyclic frequency (default: 1)\n"
    "--embedding-harmonics N  Consecutive Fourier pairs (default: 1)\n"
    "--equiangular-overlap X  Off-diagonal cosine, -1/(V-1)<=X<=1 (default: 0)\n"
    "--embedding-norm NAME  none (default), unit, rms; effective tied vectors\n"
    "--freeze-embedding     Freeze embedding parameters throughout AdamW\n"
    "--preserve-features N  Inject N code coordinates and protect them through residual blocks\n"
    "--geometry-seed N      Sphere-code seed (default: 0; grok arithmetic order uses --seed)\n"
    "--rope 0|1             Slice RoPE (default: 1)\n"
    "--qk-norm 0|1          Per-head RMS QK normalization (default: 1)\n"
    "--xsa 0|1              Exclusive projection after attention (default: 1)\n";

const char *kHelp =
    "Mesh GPT on MI355X: mesh projections, XSA, KV-cached decode, AdamW training\n"
    "Usage: mesh-gpt [train|generate|grok|init] [options]\n\n"
    "grok --help           Modular arithmetic experiments from arXiv:2201.02177v1\n"
    "--dataset PATH        UTF-8 training corpus (default: data/mesh-gpt-demo.txt)\n"
    "--output PATH         Artifacts (default: target/mesh-gpt)\n"
    "--checkpoint PATH     Load for generate; save for train and init (default: OUTPUT/model.bin)\n"
    "--width N             Channels, 2..1024 for train (default: 32)\n"
    "--heads N             Heads, 1..64, divides width; even channels/head with RoPE (default: 4)\n"
    "--layers N            Transformer blocks, 1..64 (default: 2)\n"
    "--context N           Maximum sequence length, 1..4096 (default: 32)\n"
    "--attention-depth N   Embedding/Q/K/V/output mesh depth, 1..256 (default: 4)\n"
    "--ffn-depth N         Feed-forward mesh depth, 1..256 (default: 6)\n"
    "--steps N             AdamW steps (default: 1000)\n"
    "--batch N             train: sequences per batch (default: 8, at most 131072 token rows);\n"
    "                      generate: sequences, sequence b samples with seed+b (default: 1)\n"
    "--learning-rate X     AdamW learning rate (default: 0.003)\n"
    "--weight-decay X      AdamW decay on all parameters (default: 0.01)\n"
    "--report-every N      Report interval (default: 100)\n"
    "--prompt TEXT         Generation prefix (default: 'the little robot ')\n"
    "--tokens N            New characters (default: 240)\n"
    "--temperature X       Sampling temperature, 0 is greedy (default: 0.7)\n"
    "--seed N              Initialization/data/sampling seed (default: 7)\n"
    "--device N            HIP device ordinal (default: 0)\n"
    "--config NAME         generate: synthetic seeded model: tiny, symbolic, mid, long or high\n"
    "--random-prompt LEN   With --config: LEN seeded uniform token ids as the prompt\n"
    "--prompt-file PATH    generate: read the prefix from PATH; with --batch N, N lines of\n"
    "                      equal token length, one prompt per sequence\n"
    "--init NAME           init and generate --config: reference (default, the seeded\n"
    "                      initialisation) or normal (N(0, sigma^2) weights)\n"
    "--init-sigma X        Standard deviation of --init normal (default: 0.5)\n";

// The weights of a synthetic model or a new checkpoint: the reference's
// seeded initialisation (config.rs:443-449), or N(0, sigma^2) weights drawn
// with the reference's Box-Muller normal (src/simple/numerical.rs:163-167).
std::vector<float> initial_weights(const GptConfig &config, const Options &o) {
    if (o.init == "reference") return config.initial_parameters(o.seed);
    if (o.init == "normal") return Layout::build(config).initialize_normal(config, o.seed, o.init_sigma);
    throw Error("unknown initialisation: " + o.init + "; use reference or normal");
}

// --prompt-file: the whole file is the prompt, or with --batch one line per
// sequence (the line breaks are not part of the prompts).
std::vector<std::string> prompt_lines(const Options &o) {
    const std::string text = read_file(o.prompt_file);
    if (!o.batch_set) return {text};
    std::vector<std::string> lines;
    size_t start = 0;
    while (start < text.size()) {
        size_t stop = text.find('\n', start);
        if (stop == std::string::npos) stop = text.size();
        lines.push_back(text.substr(start, stop - start));
        start = stop + 1;
    }
    if (lines.size() != o.batch)
        throw Error("prompt file must hold one line per sequence (" + std::to_string(o.batch) + "), found " +
                    std::to_string(lines.size()));
    return lines;
}

// report (mesh-gpt.rs:289-299): one stdout line and one loss.csv row.
void report(std::ofstream &history, size_t step, double train, double validation) {
    std::printf("step %6zu: train CE=%.5f, validation CE=%.5f, perplexity=%.3f\n", step, train, validation,
                std::exp(validation));
    std::fflush(stdout);
    history << format("%zu,%.9f,%.9f,%.9f\n", step, train, validation, std::exp(validation));
}

// train (mesh-gpt.rs:173-287): the demo corpus split 90/10, a seeded batch per
// step, a report every `report_every` steps and at the end, then the
// checkpoint, a sample from the trained model and the run's record.
int train(Options &o, const std::string &checkpoint) {
    const std::string text = read_file(o.dataset);
    const CharacterTokenizer tokenizer = CharacterTokenizer::from_text(text);
    GptConfig &config = o.config;
    config.vocab_size = tokenizer.vocab_size();
    config.validate();
    o.training.validate();
    if (o.prompt.empty()) throw Error("generation prompt must not be empty");
    tokenizer.encode(o.prompt);
    const TextDataset dataset(tokenizer.encode(text), config);
    const size_t C = config.context;
    if (o.batch == 0 || o.batch > kMaxRows / C) throw Error("invalid dataset batch dimensions");
    const size_t rows = C * o.batch;
    std::vector<uint32_t> ex(rows), ey(rows), x(rows), y(rows);
    dataset.batch(true, C, o.batch, 101, ex.data(), ey.data());
    MeshGpt model(int(o.device), config, o.seed);
    std::printf("Mesh GPT: blocks=%zu, width=%zu, heads=%zu, context=%zu, vocabulary=%zu, parameters=%zu\n",
                config.layers, config.width, config.heads, C, tokenizer.vocab_size(), config.parameter_count());
    auto b = [](bool v) { return v ? "true" : "false"; };
    std::printf("Meshes: Q/K/V/output depth=%zu, FFN depth=%zu; embeddings=%s, form=%s, norm=%s, protected=%zu; "
                "RoPE=%s, QK-Norm=%s, XSA=%s\n",
                config.attention_mesh_depth, config.ffn_mesh_depth, name(config.embedding),
                name(config.geometry.form), name(config.geometry.normalization), config.geometry.preserve_features,
                b(config.rope), b(config.qk_norm), b(config.xsa));
    const std::filesystem::path output(o.output);
    std::filesystem::create_directories(output);
    write_file(output / "geometry.txt", geometry_metadata(config));
    std::ofstream history(output / "loss.csv", std::ios::binary);
    if (!history) throw Error("cannot write " + (output / "loss.csv").string(), kIo);
    history << "step,train_cross_entropy,validation_cross_entropy,validation_perplexity\n";
    dataset.batch(false, C, o.batch, o.seed, x.data(), y.data());
    const double initial_train = model.cross_entropy(x.data(), y.data(), rows, C);
    const double initial_validation = model.cross_entropy(ex.data(), ey.data(), rows, C);
    report(history, 0, initial_train, initial_validation);
    AdamWOptions adam;
    adam.learning_rate = o.training.learning_rate;
    adam.weight_decay = o.training.weight_decay;
    const auto start = std::chrono::steady_clock::now();
    double sum = 0.0;
    size_t count = 0;
    for (size_t step = 1; step <= o.training.steps; ++step) {
        dataset.batch(false, C, o.batch, o.seed + step, x.data(), y.data());
        sum += model.train_batch(x.data(), y.data(), rows, C, adam);
        ++count;
        if (step % o.training.report_every == 0 || step == o.training.steps) {
            report(history, step, sum / double(count), model.cross_entropy(ex.data(), ey.data(), rows, C));
            sum = 0.0;
            count = 0;
        }
    }
    history.flush();
    const double elapsed = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
    std::printf("Training time: %.3f s\n", elapsed);
    Checkpoint saved;
    saved.config = config;
    saved.tokenizer = tokenizer;
    saved.parameters = model.parameters();
    const std::filesystem::path path(checkpoint);
    if (path.has_parent_path()) std::filesystem::create_directories(path.parent_path());
    saved.save(checkpoint);
    const std::string generated = model.generate(tokenizer, o.prompt, o.tokens, o.temperature, o.seed);
    write_file(output / "sample.txt", generated);
    const double final_validation = model.cross_entropy(ex.data(), ey.data(), rows, C);
    std::string run =
        "attention=xsa\npositions=slice_rope\nrope_base=10000\nnormalization=pre_rmsnorm\nrmsnorm_epsilon=1e-5\n"
        "rmsnorm_affine=false\nqk_norm=per_head_rmsnorm\nbias=false\nembeddings=mesh\n"
        "token_codes=signed_binary_parity_radix\nembedding_depth=attention_mesh_depth\nhead=tied_mesh_embeddings\n"
        "all_parameters=mesh_edges\n";
    run += "dataset=" + o.dataset + "\n";
    run += format("seed=%llu\nsteps=%zu\nbatch=%zu\nwidth=%zu\nheads=%zu\nlayers=%zu\ncontext=%zu\n"
                  "attention_mesh_depth=%zu\nffn_mesh_depth=%zu\nparameters=%zu\n",
                  (unsigned long long)o.seed, o.training.steps, o.batch, config.width, config.heads, config.layers,
                  C, config.attention_mesh_depth, config.ffn_mesh_depth, config.parameter_count());
    run += "learning_rate=" + display_f32(o.training.learning_rate) + "\n";
    run += "weight_decay=" + display_f32(o.training.weight_decay) + "\n";
    run += format("training_seconds=%.6f\ninitial_validation_cross_entropy=%.9f\n"
                  "final_validation_cross_entropy=%.9f\n",
                  elapsed, initial_validation, final_validation);
    write_file(output / "run.txt", run);
    std::printf("Saved checkpoint to %s\n\n%s\n", checkpoint.c_str(), generated.c_str());
    return 0;
}


// ---- grok (src/bin/mesh-gpt/grokking.rs): the modular-arithmetic experiment
// on Mesh GPT.  Answer-only AdamW training on seeded minibatches of the
// training split, a ten-update warmup, complete-split evaluations at each
// report, and the reference's artifacts.

const char *const kOperationNames[] = {"add",       "mul",       "sub",       "div",           "mixed",
                                       "square-sum", "quadratic", "quadratic-linear", "cubic-product", "cubic-mixed"};

uint32_t parse_operation(const std::string &text) {  // grokking.rs:75-93
    for (uint32_t i = 0; i < 10; ++i)
        if (text == kOperationNames[i]) return i;
    throw Error("unknown operation: " + text);
}

// Rust's Display of an f64: the shortest decimal that reads back, no exponent.
std::string display_f64(double v) {
    if (std::isnan(v)) return "NaN";
    if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
    char buf[400];
    auto res = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::fixed);
    return std::string(buf, res.ptr);
}

struct GrokOptions {
    GptConfig config;
    AdamWOptions optimizer;
    size_t modulus = 97;
    uint32_t operation = 0;
    double train_fraction = 0.5;
    size_t steps = 100000, report_every = 1000, evaluation_batch = 128, workspace_capacity = 1, qk_signs = 0;
    size_t epochs = 0, batch = 0, device = 0;
    bool has_epochs = false, has_batch = false, has_stop = false, embedding_init_unit = false, help = false;
    double stop_validation_accuracy = 0.0;
    float initialization_gain = 1.0f, embedding_output_gain = 1.0f;
    uint64_t seed = 7;
    std::string output = "target/mesh-gpt-grokking";
};

GrokOptions parse_grok(const std::vector<std::string> &args) {  // grokking.rs:44-128
    GrokOptions o;
    o.config.width = 128;
    o.config.context = 4;
    o.optimizer.learning_rate = 0.001f;
    o.optimizer.weight_decay = 1.0f;
    o.optimizer.beta2 = 0.98f;
    bool explicit_steps = false;
    for (auto it = args.cbegin(); it != args.cend(); ++it) {
        const std::string flag = *it;
        const auto end = args.cend();
        if (flag == "--modulus") o.modulus = value<size_t>(it, end, flag);
        else if (flag == "--operation") o.operation = named(it, end, flag, parse_operation);
        else if (flag == "--train-fraction") o.train_fraction = value<double>(it, end, flag);
        else if (flag == "--steps") o.steps = value<size_t>(it, end, flag), explicit_steps = true;
        else if (flag == "--epochs") o.epochs = value<size_t>(it, end, flag), o.has_epochs = true;
        else if (flag == "--batch") o.batch = value<size_t>(it, end, flag), o.has_batch = true;
        else if (flag == "--report-every") o.report_every = value<size_t>(it, end, flag);
        else if (flag == "--stop-validation-accuracy")
            o.stop_validation_accuracy = value<double>(it, end, flag), o.has_stop = true;
        else if (flag == "--eval-batch") o.evaluation_batch = value<size_t>(it, end, flag);
        else if (flag == "--workspace-cache") o.workspace_capacity = value<size_t>(it, end, flag);
        else if (flag == "--init-gain") o.initialization_gain = value<float>(it, end, flag);
        else if (flag == "--embedding-output-gain") o.embedding_output_gain = value<float>(it, end, flag);
        else if (flag == "--embedding-init-unit") o.embedding_init_unit = true;
        else if (flag == "--qk-signs") o.qk_signs = value<size_t>(it, end, flag);
        else if (flag == "--width") o.config.width = value<size_t>(it, end, flag);
        else if (flag == "--heads") o.config.heads = value<size_t>(it, end, flag);
        else if (flag == "--layers") o.config.layers = value<size_t>(it, end, flag);
        else if (flag == "--attention-depth") o.config.attention_mesh_depth = value<size_t>(it, end, flag);
        else if (flag == "--ffn-depth") o.config.ffn_mesh_depth = value<size_t>(it, end, flag);
        else if (flag == "--learning-rate") o.optimizer.learning_rate = value<float>(it, end, flag);
        else if (flag == "--weight-decay") o.optimizer.weight_decay = value<float>(it, end, flag);
        else if (flag == "--seed") o.seed = value<uint64_t>(it, end, flag);
        else if (flag == "--device") o.device = value<size_t>(it, end, flag);
        else if (flag == "--output") o.output = value<std::string>(it, end, flag);
        else if (flag == "--help" || flag == "-h") o.help = true;
        else if (!geometry_option(o.config, flag, it, end))
            throw Error("unknown grok option: " + flag + "; use grok --help");
    }
    if (explicit_steps && o.has_epochs) throw Error("choose either --epochs or --steps");
    return o;
}

const char *kGrokHelp =
    "Mesh GPT grokking: abstract-symbol modular equations from arXiv:2201.02177v1\n"
    "Usage: mesh-gpt grok [options]\n\n"
    "--operation NAME      add (default), sub, div, mixed, square-sum, quadratic,\n"
    "                      quadratic-linear, cubic-product, cubic-mixed\n"
    "--modulus P           Prime, 2..254 (default: 97)\n"
    "--train-fraction X    Fixed training fraction, 0<X<1 (default: 0.5)\n"
    "--steps N             Gradient updates (default: 100000)\n"
    "--epochs N            Complete passes over all training equations; replaces --steps\n"
    "--stop-validation-accuracy X  End at the first report with validation accuracy\n"
    "                      >=X, 0<X<=1 (default: none; train the whole budget)\n"
    "--batch N             Equations per minibatch (default: min(512, train_size/2))\n"
    "--report-every N      Evaluate both complete splits (default: 1000)\n"
    "--eval-batch N        Equations per evaluation chunk (default: 128)\n"
    "--workspace-cache N   Accepted for compatibility, 1..3: the device buffers are kept for the largest\n"
    "                      batch either way (default: 1)\n"
    "--init-gain X         Scale every initial mesh edge (default: 1)\n"
    "--embedding-output-gain X  Additional gain on the final tied-embedding layer (default: 1)\n"
    "--embedding-init-unit  Normalize table rows once before training; requires\n"
    "                      table embeddings, embedding-norm none, no protected features\n"
    "--qk-signs 0|1        Independent seeded signs on final Q/K mesh rows (default: 0)\n"
    "--learning-rate X     Maximum AdamW rate (default: 0.001; 10-step warmup)\n"
    "--weight-decay X      AdamW decay (default: 1; betas fixed at 0.9, 0.98)\n"
    "--width N             Channels, 2..1024 (default: 128)\n"
    "--heads N             Heads, 1..8; even channels/head with RoPE (default: 4)\n"
    "--layers N            Transformer blocks, 1..64 (default: 2)\n"
    "--attention-depth N   Embedding/Q/K/V/output mesh depth (default: 4)\n"
    "--ffn-depth N         Feed-forward mesh depth (default: 6)\n"
    "--embedding NAME      Tied token vectors: mesh (default) or table; the parity\n"
    "                      table starts from the seeded mesh's vectors\n"
    "--connectivity NAME   Second mesh parent: neighbor, c+1 (default), or\n"
    "                      butterfly, c+2^(layer mod floor(log2 width))\n"
    "--seed N              Model, symbol permutation, split, sampling seed (default: 7)\n"
    "--device N            HIP device ordinal (default: 0)\n"
    "--output PATH         Artifacts (default: target/mesh-gpt-grokking)\n";

// EquationSampler (grokking.rs:273-306): shuffled epochs without replacement,
// a short final batch completing each epoch.
class EquationSampler {
  public:
    EquationSampler(size_t examples, uint64_t seed) : random_(seed ^ 0x6261746368657303ULL) {
        if (examples == 0 || examples > 256 * 256) throw Error("sampler needs 1..65536 training equations");
        indices_.resize(examples);
        for (size_t i = 0; i < examples; ++i) indices_[i] = i;
        shuffle();
    }
    std::vector<size_t> sample(size_t batch) {
        if (batch == 0 || batch > indices_.size() || batch > kMaxRows / 4) throw Error("invalid equation minibatch size");
        if (position_ == indices_.size()) {
            shuffle();
            position_ = 0;
        }
        const size_t start = position_;
        position_ = std::min(start + batch, indices_.size());
        return std::vector<size_t>(indices_.begin() + start, indices_.begin() + position_);
    }

  private:
    void shuffle() {
        for (size_t end = indices_.size(); end-- > 1;) std::swap(indices_[end], indices_[random_.index(end + 1)]);
    }
    std::vector<size_t> indices_;
    Random random_;
    size_t position_ = 0;
};

// EquationDataset::symbol_label (grokking.rs:212-224)
std::string symbol_label(const EquationDataset &d, size_t token) {
    if (token == d.modulus) return kOperationNames[d.operation];
    if (token == d.modulus + 1) return "=";
    for (size_t r = 0; r < d.residue_tokens.size(); ++r)
        if (d.residue_tokens[r] == token) return std::to_string(r);
    throw Error("invalid symbol ID");
}

void validate_embedding_init_unit(const GptConfig &c, bool enabled) {  // grokking.rs:465-474
    if (enabled && (c.embedding != TokenEmbedding::Table || c.geometry.normalization != EmbeddingNorm::None ||
                    c.geometry.preserve_features != 0))
        throw Error("initial unit normalization requires table embeddings, embedding-norm none, and no protected "
                    "features");
}

// row_metrics (grokking.rs:544-558): the first maximal logit's token, and the
// f64 cross-entropy of `target` from the f32 logits.
std::pair<double, size_t> row_metrics(const float *row, size_t V, size_t target) {
    size_t prediction = 0;
    for (size_t t = 1; t < V; ++t)
        if (row[t] > row[prediction]) prediction = t;
    const double maximum = double(row[prediction]);
    double sum = 0.0;
    for (size_t t = 0; t < V; ++t) sum += std::exp(double(row[t]) - maximum);
    return {std::log(sum) + maximum - double(row[target]), prediction};
}

struct Metrics {
    double loss = 0.0, accuracy = 0.0;
};

// Logits of the answer position of equations [start, end) of a split.
template <class F>
void for_each_answer(MeshGpt &model, const EquationDataset &d, bool validation, size_t batch, F &&f) {
    const size_t count = (validation ? d.validation : d.training).size(), V = d.modulus + 2;
    std::vector<size_t> idx;
    std::vector<uint32_t> x, y;
    for (size_t start = 0; start < count; start += batch) {
        const size_t n = std::min(batch, count - start);
        idx.resize(n);
        for (size_t i = 0; i < n; ++i) idx[i] = start + i;
        x.resize(4 * n);
        y.resize(4 * n);
        d.batch(validation, idx.data(), n, x.data(), y.data());
        const std::vector<float> logits = model.logits(x.data(), 4 * n, 4, true);  // last row of each
        for (size_t i = 0; i < n; ++i) f(start + i, logits.data() + i * V, size_t(y[4 * i + 3]));
    }
}

Metrics evaluate(MeshGpt &model, const EquationDataset &d, bool validation, size_t batch) {  // grokking.rs:560-586
    const size_t count = (validation ? d.validation : d.training).size(), V = d.modulus + 2;
    double loss = 0.0;
    size_t correct = 0;
    for_each_answer(model, d, validation, batch, [&](size_t, const float *row, size_t target) {
        const auto [ce, prediction] = row_metrics(row, V, target);
        loss += ce;
        correct += prediction == target;
    });
    return {loss / double(count), double(correct) / double(count)};
}

struct Thresholds {
    long training = -1, validation = -1;
};

std::string observed(long step) { return step < 0 ? "not_reached" : std::to_string(step); }

double weight_norm(const std::vector<float> &p) {
    double s = 0.0;
    for (float x : p) s += double(x) * double(x);
    return std::sqrt(s);
}

// record (grokking.rs:588-640): complete-split metrics, a loss.csv row, the
// checkpoint, and the report line; returns the validation accuracy.
double record(std::ofstream &history, MeshGpt &model, const EquationDataset &d, const CharacterTokenizer &tok,
              size_t eval_batch, const std::filesystem::path &dir, size_t step, size_t trained, float lr,
              double elapsed, Thresholds &th) {
    const Metrics train = evaluate(model, d, false, eval_batch), valid = evaluate(model, d, true, eval_batch);
    if (train.accuracy >= 0.99 && th.training < 0) th.training = long(step);
    if (valid.accuracy >= 0.99 && th.validation < 0) th.validation = long(step);
    Checkpoint saved;
    saved.config = model.config();
    saved.tokenizer = tok;
    saved.parameters = model.parameters();
    const size_t n_train = d.training.size();
    history << format("%zu,%zu,%zu,%zu,%.9f,%.9f,%.9f,%.9f,%.9f,%.9f,%.6f\n", step, trained, trained / n_train,
                      trained % n_train, train.loss, valid.loss, train.accuracy, valid.accuracy,
                      weight_norm(saved.parameters), double(lr), elapsed);
    history.flush();
    saved.save((dir / "model.bin").string());
    std::printf("step %7zu: train CE=%.5f accuracy=%.2f%%; validation CE=%.5f accuracy=%.2f%%\n", step, train.loss,
                100.0 * train.accuracy, valid.loss, 100.0 * valid.accuracy);
    std::fflush(stdout);
    return valid.accuracy;
}

void write_embeddings(const std::filesystem::path &path, MeshGpt &model, const EquationDataset &d) {
    const size_t W = model.config().width, V = model.config().vocab_size;
    const std::vector<float> e = model.token_embeddings();
    std::string s = "token_id,symbol";
    for (size_t c = 0; c < W; ++c) s += ",c" + std::to_string(c);
    s += "\n";
    for (size_t t = 0; t < V; ++t) {
        s += std::to_string(t) + "," + symbol_label(d, t);
        for (size_t c = 0; c < W; ++c) s += format(",%.9f", double(e[t * W + c]));
        s += "\n";
    }
    write_file(path, s);
}

int grok(const std::vector<std::string> &args) {
    GrokOptions o = parse_grok(args);
    if (o.help) {
        std::cout << kGrokHelp << "\n" << kGeometryHelp;
        return 0;
    }
    GptConfig &config = o.config;
    if (config.width > 1024) throw Error("grokking requires width <=1024");
    if (o.steps == 0 || o.report_every == 0 || o.evaluation_batch == 0)
        throw Error("steps, report interval, and evaluation batch must be positive");
    for (float gain : {o.initialization_gain, o.embedding_output_gain})
        if (!std::isfinite(gain) || gain <= 0.0f) throw Error("initialization gains must be finite and positive");
    if (o.workspace_capacity < 1 || o.workspace_capacity > 3) throw Error("workspace capacity must be in 1..3");
    if (o.has_stop && !(o.stop_validation_accuracy > 0.0 && o.stop_validation_accuracy <= 1.0))
        throw Error("validation stop accuracy must be in (0, 1]");
    if (o.qk_signs > 1) throw Error("Q/K sign initialization must be 0 or 1");
    o.optimizer.validate();
    const EquationDataset dataset = EquationDataset::build(o.modulus, o.operation, o.train_fraction, o.seed);
    const CharacterTokenizer tokenizer = dataset.tokenizer();
    config.vocab_size = tokenizer.vocab_size();
    if (config.geometry.order != EmbeddingOrder::Token) {
        config.geometry.modulus = o.modulus;
        config.geometry.seed = o.seed;
    }
    config.validate();
    // The reference's grok model type holds at most 8 heads (grokking.rs:20).
    if (config.heads > 8) throw Error("grokking requires at most 8 heads");
    validate_embedding_init_unit(config, o.embedding_init_unit);
    const size_t n_train = dataset.training.size(), n_valid = dataset.validation.size();
    const size_t batch = o.has_batch ? o.batch : std::min<size_t>(512, n_train / 2);
    EquationSampler(n_train, o.seed).sample(batch);  // validates the minibatch size
    if (o.has_epochs) {  // epoch_steps (grokking.rs:504-513)
        if (o.epochs == 0 || batch == 0) throw Error("epochs, training examples, and batch size must be positive");
        const size_t per = (n_train + batch - 1) / batch;
        if (o.epochs > SIZE_MAX / per) throw Error("epoch budget exceeds the supported update count");
        o.steps = o.epochs * per;
    }
    EquationSampler sampler(n_train, o.seed);
    MeshGpt model(int(o.device), config, o.seed);
    if (o.initialization_gain != 1.0f || o.embedding_output_gain != 1.0f || o.qk_signs == 1 ||
        o.embedding_init_unit) {
        // grokking.rs:221-283: adjust the mesh-embedding initialisation; a table
        // then stores the adjusted mesh's vectors.
        GptConfig mesh = config;
        mesh.embedding = TokenEmbedding::Mesh;
        std::vector<float> p = mesh.initial_parameters(o.seed);
        for (float &v : p) v *= o.initialization_gain;
        const size_t W = config.width, A = config.attention_mesh_depth, F = config.ffn_mesh_depth;
        const size_t emb_end = 2 * W * A;
        for (size_t i = emb_end - 2 * W; i < emb_end; ++i) p[i] *= o.embedding_output_gain;
        if (o.qk_signs == 1) {
            uint64_t state = o.seed ^ 0x514b5349474e5331ULL;
            const size_t mesh_size = 2 * W * A, block_size = 2 * W * (4 * A + F);
            for (size_t blk = 0; blk < config.layers; ++blk)
                for (size_t proj = 0; proj < 2; ++proj) {
                    const size_t end = mesh_size + blk * block_size + (proj + 1) * mesh_size;
                    for (size_t i = end - 2 * W; i < end; i += 2) {
                        // SplitMix64 on its own stream (src/mesh.rs:267-274)
                        state += 0x9e3779b97f4a7c15ULL;
                        uint64_t bits = state;
                        bits = (bits ^ (bits >> 30)) * 0xbf58476d1ce4e5b9ULL;
                        bits = (bits ^ (bits >> 27)) * 0x94d049bb133111ebULL;
                        bits ^= bits >> 31;
                        const float sign = bits >> 63 == 0 ? 1.0f : -1.0f;
                        p[i] *= sign;
                        p[i + 1] *= sign;
                    }
                }
        }
        if (config.embedding == TokenEmbedding::Table) {
            p = tabulate_embedding(mesh, p);
            if (config.geometry.form != EmbeddingForm::Parity) {
                const std::vector<float> codes = token_codes(config);
                for (size_t i = 0; i < config.embedding_parameter_count(); ++i)
                    p[i] = codes[i] * o.initialization_gain * o.embedding_output_gain;
            }
        }
        if (o.embedding_init_unit) {  // normalize_table_initialization (grokking.rs:476-502)
            std::vector<double> norms(config.vocab_size);
            for (size_t t = 0; t < config.vocab_size; ++t) {
                double s = 0.0;
                for (size_t c = 0; c < W; ++c) s += double(p[t * W + c]) * double(p[t * W + c]);
                norms[t] = std::sqrt(s);
                if (!std::isfinite(norms[t]) || norms[t] < 1e-12)
                    throw Error("initial unit normalization requires finite, nonzero table rows");
            }
            for (size_t t = 0; t < config.vocab_size; ++t)
                for (size_t c = 0; c < W; ++c) p[t * W + c] = float(double(p[t * W + c]) / norms[t]);
        }
        model.set_parameters(p.data(), p.size());
    }
    const std::filesystem::path dir(o.output);
    std::filesystem::create_directories(dir);
    {  // write_dataset (grokking.rs:642-676)
        std::string e = "split,pair_id,a,b,answer,input_a_id,operator_id,input_b_id,equals_id,target_id\n";
        for (bool validation : {false, true})
            for (const auto &q : validation ? dataset.validation : dataset.training)
                e += format("%s,%zu,%zu,%zu,%zu,%u,%zu,%u,%zu,%u\n", validation ? "validation" : "train",
                            q.a * dataset.modulus + q.b, q.a, q.b, q.answer, dataset.residue_tokens[q.a],
                            dataset.modulus, dataset.residue_tokens[q.b], dataset.modulus + 1,
                            dataset.residue_tokens[q.answer]);
        write_file(dir / "equations.csv", e);
        std::string sy = "token_id,symbol\n";
        for (size_t t = 0; t < tokenizer.vocab_size(); ++t) sy += std::to_string(t) + "," + symbol_label(dataset, t) + "\n";
        write_file(dir / "symbols.csv", sy);
    }
    auto b = [](bool v) { return v ? "true" : "false"; };
    std::string run = "paper=https://arxiv.org/abs/2201.02177v1\nstatus=running\nmodel=mesh_gpt\n";
    run += std::string("operation=") + kOperationNames[o.operation] + "\n";
    run += format("modulus=%zu\n", o.modulus);
    run += "train_fraction=" + display_f64(o.train_fraction) + "\n";
    run += format("training_equations=%zu\nvalidation_equations=%zu\nseed=%llu\n", n_train, n_valid,
                  (unsigned long long)o.seed);
    run += "abstract_symbol_permutation=true\nloss=answer_only\ncontext=4\n";
    run += format("width=%zu\nheads=%zu\nlayers=%zu\nattention_mesh_depth=%zu\nffn_mesh_depth=%zu\nparameters=%zu\n"
                  "embedding_parameters=%zu\n",
                  config.width, config.heads, config.layers, config.attention_mesh_depth, config.ffn_mesh_depth,
                  config.parameter_count(), config.embedding_parameter_count());
    run += std::string("all_parameters=") +
           (config.embedding == TokenEmbedding::Mesh ? "mesh_edges" : "mesh_edges_and_token_table") + "\n";
    run += std::string("attention=") + (config.xsa ? "xsa" : "softmax") + "\n";
    run += std::string("positions=") + (config.rope ? "slice_rope" : "none") + "\n";
    run += "normalization=pre_rmsnorm\n";
    run += std::string("qk_norm=") + (config.qk_norm ? "per_head_rmsnorm" : "none") + "\n";
    run += "rmsnorm_affine=false\nbias=false\n";
    run += std::string("embeddings=") + name(config.embedding) + "\n";
    run += std::string("mesh_connectivity=") + name(config.connectivity) + "\n";
    run += "betas=0.9,0.98\nepsilon=1e-8\n";
    run += "learning_rate=" + display_f32(o.optimizer.learning_rate) + "\n";
    run += "weight_decay=" + display_f32(o.optimizer.weight_decay) + "\n";
    run += format("warmup_steps=10\nbatch=%zu\nsteps=%zu\nreport_every=%zu\n", batch, o.steps, o.report_every);
    run += "evaluation=complete_splits\ncheckpoint=weights_only\n";
    run += geometry_metadata(config);
    run += "requested_epochs=" + (o.has_epochs ? std::to_string(o.epochs) : std::string("none")) + "\n";
    run += format("steps_per_epoch=%zu\n", (n_train + batch - 1) / batch);
    run += "epoch_definition=one_visit_to_every_training_equation\nepoch_tail=short_batch\n";
    run += "stop_validation_accuracy=" + (o.has_stop ? display_f64(o.stop_validation_accuracy) : std::string("none")) +
           "\n";
    run += format("evaluation_batch=%zu\n", o.evaluation_batch);
    run += "initialization_gain=" + display_f32(o.initialization_gain) + "\n";
    run += "embedding_output_gain=" + display_f32(o.embedding_output_gain) + "\n";
    run += std::string("embedding_init_unit=") + b(o.embedding_init_unit) + "\n";
    run += format("qk_signs=%zu\nworkspace_capacity=%zu\n", o.qk_signs, o.workspace_capacity);
    write_file(dir / "run.txt", run);
    std::printf("Mesh GPT grokking: %s mod %zu, train=%zu, validation=%zu, batch=%zu, parameters=%zu\n",
                kOperationNames[o.operation], o.modulus, n_train, n_valid, batch, config.parameter_count());
    std::printf("Answer-only loss; AdamW beta2=0.98, decay=%s, warmup=10; continuing for %zu updates%s\n",
                display_f32(o.optimizer.weight_decay).c_str(), o.steps,
                o.has_stop ? (" or validation accuracy >=" + display_f64(o.stop_validation_accuracy)).c_str() : "");
    std::ofstream history(dir / "loss.csv", std::ios::binary);
    if (!history) throw Error("cannot write " + (dir / "loss.csv").string(), kIo);
    history << "step,training_examples_seen,completed_epochs,examples_in_partial_epoch,train_cross_entropy,"
               "validation_cross_entropy,train_accuracy,validation_accuracy,weight_l2,learning_rate,elapsed_seconds\n";
    const auto start = std::chrono::steady_clock::now();
    auto elapsed = [&] { return std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count(); };
    Thresholds th;
    double validation_accuracy =
        record(history, model, dataset, tokenizer, o.evaluation_batch, dir, 0, 0, 0.0f, elapsed(), th);
    std::filesystem::copy_file(dir / "model.bin", dir / "initial-model.bin",
                               std::filesystem::copy_options::overwrite_existing);
    write_embeddings(dir / "initial-embeddings.csv", model, dataset);
    auto reached = [&](double acc) { return o.has_stop && acc >= o.stop_validation_accuracy; };
    size_t step = 0, trained = 0;
    std::vector<uint32_t> x, y;
    while (step < o.steps && !reached(validation_accuracy)) {
        ++step;
        const std::vector<size_t> idx = sampler.sample(batch);
        x.resize(4 * idx.size());
        y.resize(4 * idx.size());
        dataset.batch(false, idx.data(), idx.size(), x.data(), y.data());
        AdamWOptions opt = o.optimizer;  // warmed_optimizer (grokking.rs:515-518)
        opt.learning_rate *= float(std::min<size_t>(step, 10)) / 10.0f;
        model.train_batch(x.data(), y.data(), x.size(), 4, opt);
        trained += idx.size();
        if (step % o.report_every == 0 || step == o.steps)
            validation_accuracy = record(history, model, dataset, tokenizer, o.evaluation_batch, dir, step, trained,
                                         opt.learning_rate, elapsed(), th);
    }
    const char *stop_reason = reached(validation_accuracy) ? "validation_accuracy" : "update_budget";
    write_embeddings(dir / "embeddings.csv", model, dataset);
    {  // write_predictions (grokking.rs:697-733)
        std::string pr = "split,a,b,answer,prediction,correct,cross_entropy\n";
        const size_t V = dataset.modulus + 2;
        for (bool validation : {false, true}) {
            const auto &split = validation ? dataset.validation : dataset.training;
            for_each_answer(model, dataset, validation, o.evaluation_batch,
                            [&](size_t i, const float *row, size_t target) {
                                const auto [ce, prediction] = row_metrics(row, V, target);
                                const auto &q = split[i];
                                pr += format("%s,%zu,%zu,%zu,", validation ? "validation" : "train", q.a, q.b,
                                             q.answer) +
                                      symbol_label(dataset, prediction) + format(",%d,%.9f\n", int(prediction == target), ce);
                            });
        }
        write_file(dir / "predictions.csv", pr);
    }
    std::string done = run;
    done.replace(done.find("status=running"), 14, "status=complete");
    done += format("elapsed_seconds=%.6f\nstop_reason=%s\ncompleted_steps=%zu\ntraining_examples_seen=%zu\n"
                   "completed_epochs=%zu\nexamples_in_partial_epoch=%zu\n",
                   elapsed(), stop_reason, step, trained, trained / n_train, trained % n_train);
    done += "first_recorded_train_99_step=" + observed(th.training) + "\n";
    done += "first_recorded_validation_99_step=" + observed(th.validation) + "\n";
    write_file(dir / "run.txt", done);
    std::printf("Saved model, split, symbols, embeddings, predictions, and learning curves to %s\n",
                o.output.c_str());
    std::printf("First recorded accuracy >=99%%: train=%s, validation=%s\n", observed(th.training).c_str(),
                observed(th.validation).c_str());
    std::printf("Stopped after %zu updates: %s\n", step, stop_reason);
    return 0;
}

int run(int argc, char **argv) {
    if (argc > 1 && std::string(argv[1]) == "grok") return grok(std::vector<std::string>(argv + 2, argv + argc));
    Options o = parse(argc, argv);
    if (o.help) {
        std::cout << kHelp << "\n" << kGeometryHelp;
        return 0;
    }
    if (!std::isfinite(o.temperature) || o.temperature < 0.0f)
        throw Error("temperature must be finite and nonnegative");
    const std::string checkpoint = o.checkpoint.empty() ? o.output + "/model.bin" : o.checkpoint;
    if (o.command == "train") {
        if (!o.batch_set) o.batch = 8;  // the training default (mesh-gpt.rs:54)
        return train(o, checkpoint);
    }
    if (o.command == "generate") {
        GptConfig config;
        CharacterTokenizer tokenizer;
        std::vector<float> parameters;
        std::vector<uint32_t> prompt;
        if (!o.synthetic.empty()) {
            config = named_config(o.synthetic);
            std::vector<uint32_t> chars(config.vocab_size);
            for (size_t i = 0; i < chars.size(); ++i) chars[i] = uint32_t(config.vocab_size == 64 ? 0x20 + i : i);
            tokenizer = CharacterTokenizer::from_characters(chars);
            parameters = initial_weights(config, o);
            if (o.random_prompt) {
                Random r(o.seed);
                for (size_t i = 0; i < o.batch * o.random_prompt; ++i)
                    prompt.push_back(uint32_t(r.index(config.vocab_size)));
            }
        } else {
            Checkpoint saved = Checkpoint::load(checkpoint);
            config = saved.config;
            tokenizer = saved.tokenizer;
            parameters = std::move(saved.parameters);
        }
        MeshGpt model(int(o.device), config, o.seed, o.batch);
        model.set_parameters(parameters.data(), parameters.size());
        std::vector<std::string> texts;
        if (!o.prompt_file.empty() && prompt.empty()) texts = prompt_lines(o);
        if (prompt.empty() && !o.batch_set) {
            const std::string &text = texts.empty() ? o.prompt : texts[0];
            std::cout << model.generate(tokenizer, text, o.tokens, o.temperature, o.seed) << "\n";
            return 0;
        }
        if (prompt.empty() && !texts.empty()) {
            size_t p = 0;
            for (size_t b = 0; b < o.batch; ++b) {
                std::vector<uint32_t> one = tokenizer.encode(texts[b]);
                if (one.empty()) throw Error("generation prompt must not be empty");
                if (b > 0 && one.size() != p) throw Error("batched prompts must have equal token lengths");
                p = one.size();
                prompt.insert(prompt.end(), one.begin(), one.end());
            }
        }
        if (prompt.empty()) {
            std::vector<uint32_t> one = tokenizer.encode(o.prompt);
            if (one.empty()) throw Error("generation prompt must not be empty");
            for (size_t b = 0; b < o.batch; ++b) prompt.insert(prompt.end(), one.begin(), one.end());
        }
        const size_t p = prompt.size() / o.batch, n = p + o.tokens;
        std::vector<uint32_t> out(o.batch * n);
        model.generate_tokens(prompt.data(), o.batch, p, o.tokens, o.temperature, o.seed, out.data());
        for (size_t b = 0; b < o.batch; ++b) std::cout << tokenizer.decode(out.data() + b * n, n) << "\n";
        return 0;
    }
    if (o.command == "init") {
        std::FILE *f = std::fopen(o.dataset.c_str(), "rb");
        if (!f) throw Error("cannot open dataset " + o.dataset, kIo);
        std::string text;
        char buf[4096];
        size_t got;
        while ((got = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, got);
        std::fclose(f);
        Checkpoint ck;
        ck.tokenizer = CharacterTokenizer::from_text(text);
        ck.config = o.config;
        ck.config.vocab_size = ck.tokenizer.vocab_size();
        ck.parameters = initial_weights(ck.config, o);
        ck.save(checkpoint);
        std::cout << "Saved seed-" << o.seed << " checkpoint to " << checkpoint << "\n";
        return 0;
    }
    if (o.command == "verify")
        throw Error("the verify command is not part of this CLI, which does not link the CPU oracle: run python "
                    "tests/verify.py (the reference's model checks, GPU against the oracle)");
    if (o.command == "grok-simple")
        throw Error("the grok-simple command is not part of this build; it provides train, generate and grok");
    throw Error("unknown command: " + o.command + "; use train, generate, grok or init");
}

}  // namespace

int main(int argc, char **argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception &e) {
        // A Rust main returning Err prints the error's Debug form.
        std::cerr << "Error: \"" << e.what() << "\"\n";
        return 1;
    }
}
