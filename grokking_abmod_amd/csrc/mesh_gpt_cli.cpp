// mesh-gpt: the reference's `mesh-gpt generate` command (src/bin/mesh-gpt.rs:
// 29-164) on the MI355X library, with the same flags, defaults, output and
// error text.  Extensions: --batch N (N sequences, seeds seed..seed+N-1, one
// line each), --config NAME with --random-prompt LEN (a seeded synthetic model
// and prompt, no checkpoint), and `init` (write a seeded checkpoint).
#include <cmath>
#include <cstdio>
#include <cstdlib>
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
        else if (flag == "--embedding") o.config.embedding = parse_embedding(value<std::string>(it, end, flag));
        else if (flag == "--connectivity")
            o.config.connectivity = parse_connectivity(value<std::string>(it, end, flag));
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
        else if (flag == "--help" || flag == "-h") o.help = true;
        else throw Error("unknown option: " + flag + "; use --help");
    }
    return o;
}

const char *kHelp =
    "Mesh GPT generate on MI355X: mesh projections, XSA, KV-cached decode\n"
    "Usage: mesh-gpt [generate|init] [options]\n\n"
    "--checkpoint PATH     Load for generate; write for init (default: OUTPUT/model.bin)\n"
    "--output PATH         Artifacts (default: target/mesh-gpt)\n"
    "--prompt TEXT         Generation prefix (default: 'the little robot ')\n"
    "--tokens N            New characters (default: 240)\n"
    "--temperature X       Sampling temperature, 0 is greedy (default: 0.7)\n"
    "--seed N              Initialization/sampling seed (default: 7)\n"
    "--device N            HIP device ordinal (default: 0)\n"
    "--batch N             Sequences; sequence b samples with seed+b (default: 1)\n"
    "--config NAME         Synthetic seeded model: tiny, symbolic, mid, long or high\n"
    "--random-prompt LEN   With --config: LEN seeded uniform token ids as the prompt\n"
    "init: --dataset PATH (tokenizer corpus), --width --heads --layers --context\n"
    "      --attention-depth --ffn-depth --embedding mesh|table --connectivity neighbor|butterfly\n";

int run(int argc, char **argv) {
    Options o = parse(argc, argv);
    if (o.help) {
        std::cout << kHelp;
        return 0;
    }
    if (!std::isfinite(o.temperature) || o.temperature < 0.0f)
        throw Error("temperature must be finite and nonnegative");
    const std::string checkpoint = o.checkpoint.empty() ? o.output + "/model.bin" : o.checkpoint;
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
            parameters = config.initial_parameters(o.seed);
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
        if (prompt.empty() && !o.batch_set) {
            std::cout << model.generate(tokenizer, o.prompt, o.tokens, o.temperature, o.seed) << "\n";
            return 0;
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
        ck.parameters = ck.config.initial_parameters(o.seed);
        ck.save(checkpoint);
        std::cout << "Saved seed-" << o.seed << " checkpoint to " << checkpoint << "\n";
        return 0;
    }
    if (o.command == "train" || o.command == "grok" || o.command == "grok-simple" || o.command == "verify")
        throw Error("the " + o.command +
                    " command is not part of this build; it provides generate (parity checks live in tests/)");
    throw Error("unknown command: " + o.command + "; use generate or init");
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
