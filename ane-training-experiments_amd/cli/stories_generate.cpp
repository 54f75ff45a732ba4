// stories-generate — command-line decoder over libstories_hip.so, the C++ host counterpart
// of cmd/stories-generate-go/main.go. Same flags and output lines; the decode itself runs
// on the GPU through the C ABI (include/stories_hip.h).
//
//   stories-generate [-model stories110M.bin] [-tokenizer tokenizer.bin] [-prompt-ids 1,2]
//                    [-max-new 64] [-temperature 0.8] [-seed N] [-seq 256] [-ane]
//
// Flags beyond the reference's (all optional):
//   -shape stories110m|qwen3-0.6b   model shape when no -model file is given
//   -dtype fp16|bf16                weight storage (default fp16; bf16 for qwen3-0.6b)
//   -kv f32|f16|bf16                KV-cache storage
//   -synthetic-seed S, -synthetic-std X
//                                   N(0, X) weights keyed by S (the library's sh_synth_normal
//                                   streams) when no -model file is given
//   -train                          with -bench-steps: time the training Step (sh_trainer_step)
//                                   at -seq tokens over a synthetic stream (-prompt-seed),
//                                   -lr, window seed -seed; one JSON object
//   -layers N                       with synthetic weights: only the first N layers of the
//                                   shape (per-layer kernels unchanged; for short profiles)
//   -prompt-len N, -prompt-seed S   a synthetic prompt of N uniform ids instead of -prompt-ids
//   -bench-steps K, -bench-warmup W greedy decode W untimed + K timed times and print one
//                                   JSON object (device times, bytes, tokens) instead of text
//   -inspect                        load the model file, print its header and per-tensor
//                                   sums as JSON, touch no GPU
//   -detokenize 5,6,7               print text= for these ids with -tokenizer, touch no GPU
//   -copy-calibrate BYTES           with -bench-steps: first time the library's plain copy
//                                   kernel over BYTES and report its GB/s
//   -read-calibrate BYTES           with -bench-steps: the same for its read-only kernel
//   -batch B                        with -bench-steps: B synthetic prompts of -prompt-len ids
//                                   (-prompt-seed) decoded together (sh_batch_greedy_decode);
//                                   the JSON object reports the prefill and per-step times
//   -eval-logits                    with -bench-steps: time sh_prefill_logits (the storiesane
//                                   EvalLogits forward) over the -prompt-len synthetic ids and
//                                   report device times and the forward's FLOPs
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <map>
#include <string>
#include <vector>

#include "llama2_file.hpp"
#include "stories_hip.h"

namespace {

[[noreturn]] void fatalf(const char *fmt, const std::string &a = "") {
    fprintf(stderr, fmt, a.c_str());
    fputc('\n', stderr);
    exit(1);
}

std::string lib_error() {
    char buf[1024];
    sh_last_error(buf, sizeof buf);
    return buf;
}

// Go flag package syntax: -name value, -name=value, --name; booleans take no value.
struct Flags {
    std::map<std::string, std::string> v;
    std::map<std::string, bool> is_bool;
    void def(const char *name, const char *dflt, bool boolean = false) {
        v[name] = dflt;
        is_bool[name] = boolean;
    }
    void parse(int argc, char **argv) {
        for (int i = 1; i < argc; i++) {
            std::string a = argv[i];
            if (a.size() < 2 || a[0] != '-') fatalf("unexpected argument %s", a);
            a = a.substr(a[1] == '-' ? 2 : 1);
            std::string val;
            const size_t eq = a.find('=');
            const bool has_eq = eq != std::string::npos;
            if (has_eq) {
                val = a.substr(eq + 1);
                a = a.substr(0, eq);
            }
            if (!v.count(a)) fatalf("flag provided but not defined: -%s", a);
            if (is_bool[a]) {
                v[a] = has_eq ? val : "true";
            } else {
                if (!has_eq) {
                    if (i + 1 >= argc) fatalf("flag needs an argument: -%s", a);
                    val = argv[++i];
                }
                v[a] = val;
            }
        }
    }
    std::string s(const char *n) const { return v.at(n); }
    long long i(const char *n) const { return strtoll(v.at(n).c_str(), nullptr, 10); }
    double f(const char *n) const { return strtod(v.at(n).c_str(), nullptr); }
    bool b(const char *n) const { return v.at(n) == "true" || v.at(n) == "1"; }
};

// main.go:121-142 parseTokenList: empty -> [1]; blanks skipped.
std::vector<int32_t> parse_token_list(const std::string &s) {
    std::vector<int32_t> out;
    size_t p = 0;
    int idx = 0;
    while (p <= s.size()) {
        size_t q = s.find(',', p);
        if (q == std::string::npos) q = s.size();
        std::string t = s.substr(p, q - p);
        const size_t a = t.find_first_not_of(" \t\n"), b = t.find_last_not_of(" \t\n");
        t = a == std::string::npos ? "" : t.substr(a, b - a + 1);
        if (!t.empty()) {
            char *end = nullptr;
            const long v = strtol(t.c_str(), &end, 10);
            if (*end) fatalf("parse prompt tokens: token[%s] is not an integer",
                             std::to_string(idx) + "]=\"" + t);
            out.push_back((int32_t)v);
        }
        idx++;
        p = q + 1;
    }
    if (out.empty()) out.push_back(1);
    return out;
}

// Host-side sampler for temperature > 1e-6: the inverse-CDF rule of infer.go:347-371 over
// float64 exp terms. Uniform draws come from splitmix64 (53-bit doubles) seeded by -seed;
// Go's math/rand stream is not reproduced, so sampled ids differ from the reference's.
struct Sampler {
    uint64_t state;
    double uniform() {
        uint64_t z = (state += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        return (double)(z >> 11) * (1.0 / 9007199254740992.0);
    }
    int sample(const float *logits, int n, float temperature) {
        float mx = logits[0];
        for (int i = 1; i < n; i++)
            if (logits[i] > mx) mx = logits[i];
        const double inv_t = (double)(1.0f / temperature);
        double total = 0;
        for (int i = 0; i < n; i++) total += exp(((double)logits[i] - (double)mx) * inv_t);
        const double target = uniform() * total;
        double acc = 0;
        for (int i = 0; i < n; i++) {
            acc += exp(((double)logits[i] - (double)mx) * inv_t);
            if (acc >= target) return i;
        }
        return n - 1;
    }
};

std::string join_ints(const std::vector<int32_t> &v) {
    std::string s;
    for (size_t i = 0; i < v.size(); i++) {
        if (i) s += ",";
        s += std::to_string(v[i]);
    }
    return s;
}

std::string json_escape(const std::string &s) {
    std::string o;
    for (char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += c;
        } else if ((unsigned char)c < 0x20) {
            char b[8];
            snprintf(b, sizeof b, "\\u%04x", (unsigned char)c);
            o += b;
        } else {
            o += c;
        }
    }
    return o;
}

// Go's time.Duration.Round(time.Millisecond).String() for the elapsed field.
std::string go_duration(double seconds) {
    const long long ms = llround(seconds * 1e3);
    char b[64];
    if (ms < 1000) snprintf(b, sizeof b, "%lldms", ms);
    else if (ms < 60000) snprintf(b, sizeof b, "%.3gs", ms / 1e3);
    else snprintf(b, sizeof b, "%lldm%.3gs", ms / 60000, (ms % 60000) / 1e3);
    return b;
}

void synth_weights(const sh_config &c, uint64_t seed, float std_, stories::HostWeights &w) {
    w.resize(c);
    for (int l = 0; l < c.n_layers; l++) {
        stories::HostLayer &L = w.layers[l];
        std::vector<float> *mats[7] = {&L.wq, &L.wk, &L.wv, &L.wo, &L.w1, &L.w2, &L.w3};
        for (int k = 0; k < 7; k++)
            if (sh_synth_normal(mats[k]->data(), mats[k]->size(), seed, 16 * (uint64_t)(l + 1) + k, std_))
                fatalf("synthetic weights: %s", lib_error());
    }
    if (sh_synth_normal(w.embed.data(), w.embed.size(), seed, 1, std_))
        fatalf("synthetic weights: %s", lib_error());
    if (!c.tied_embed && sh_synth_normal(w.cls.data(), w.cls.size(), seed, 2, std_))
        fatalf("synthetic weights: %s", lib_error());
}

sh_model *open_model(const sh_config &c, int dtype, const stories::HostWeights &w) {
    sh_model *m = sh_model_create(&c, dtype);
    if (!m) fatalf("decode: %s", lib_error());
    for (int l = 0; l < c.n_layers; l++) {
        const stories::HostLayer &L = w.layers[l];
        if (sh_model_upload_layer(m, l, L.wq.data(), L.wk.data(), L.wv.data(), L.wo.data(),
                                  L.w1.data(), L.w2.data(), L.w3.data(), L.rms_att.data(),
                                  L.rms_ffn.data(), c.qk_norm ? L.q_norm.data() : nullptr,
                                  c.qk_norm ? L.k_norm.data() : nullptr))
            fatalf("decode: %s", lib_error());
    }
    if (sh_model_upload_globals(m, w.embed.data(), w.rms_final.data(),
                                c.tied_embed ? nullptr : w.cls.data()))
        fatalf("decode: %s", lib_error());
    return m;
}

struct DecodeResult {
    std::vector<int32_t> tokens;
    int prompt_length = 0;
    bool stopped_eos = false;
    double gpu_ms = 0;   // device time of the forwards
    double bytes = 0;    // their algorithmic bytes
};

// (*Decoder).Decode (infer.go:136-202). Greedy runs entirely on the device; a sampled
// decode feeds the prompt on the device and draws each id on the host from the logits.
DecodeResult decode(sh_model *m, const sh_config &c, const std::vector<int32_t> &prompt_in,
                    int max_new, float temperature, Sampler &rng) {
    DecodeResult r;
    if (max_new <= 0) max_new = 64;
    if (temperature < 0) temperature = 0;
    // device time and algorithmic bytes of every token forward (sh_stats after each call; a
    // greedy decode's prompt forward is reported apart, as prefill_ms, and its bytes are not
    // counted, so its time is left out too)
    auto account = [&]() {
        sh_timing t{};
        if (sh_stats(m, &t) == 0) {
            r.gpu_ms += t.gpu_ms - t.prefill_ms;
            r.bytes += t.bytes_per_forward_mean * (double)t.forwards;
        }
    };
    if (temperature <= 1e-6f) {
        std::vector<int32_t> out(c.max_seq);
        int32_t n = 0, eos = 0;
        if (sh_greedy_decode(m, prompt_in.data(), (int32_t)prompt_in.size(), max_new, out.data(),
                             &n, &eos))
            fatalf("decode: %s", lib_error());
        account();
        std::vector<int32_t> p = prompt_in.empty() ? std::vector<int32_t>{1} : prompt_in;
        r.prompt_length = (int)std::min(p.size(), (size_t)c.max_seq);
        r.tokens.assign(out.begin(), out.begin() + n);
        r.stopped_eos = eos != 0;
        return r;
    }
    std::vector<int32_t> prompt = prompt_in.empty() ? std::vector<int32_t>{1} : prompt_in;
    if ((int)prompt.size() > c.max_seq) prompt.erase(prompt.begin(), prompt.end() - c.max_seq);
    for (size_t i = 0; i < prompt.size(); i++)
        if (prompt[i] < 0 || prompt[i] >= c.vocab)
            fatalf("decode: %s", "prompt token[" + std::to_string(i) + "]=" +
                                     std::to_string(prompt[i]) + " out of range");
    if (sh_reset_cache(m)) fatalf("decode: %s", lib_error());
    r.tokens = prompt;
    r.prompt_length = (int)prompt.size();
    for (size_t pos = 0; pos + 1 < prompt.size(); pos++) {
        if (sh_decode_step(m, prompt[pos], (int32_t)pos, nullptr, nullptr))
            fatalf("decode: %s", lib_error());
        account();
    }
    std::vector<float> logits(c.vocab);
    for (int step = 0; step < max_new && (int)r.tokens.size() < c.max_seq; step++) {
        const int pos = (int)r.tokens.size() - 1;
        if (sh_decode_step(m, r.tokens[pos], pos, logits.data(), nullptr))
            fatalf("decode: %s", lib_error());
        account();
        const int next = rng.sample(logits.data(), c.vocab, temperature);
        r.tokens.push_back(next);
        if (next == 2) {
            r.stopped_eos = true;
            break;
        }
    }
    return r;
}

// (*Engine).Decode (ane/storiesane/decode.go:18-94): every step evaluates the whole window
// of the last `seq` tokens, left-padded with BOS (fillDecodeWindow, decode.go:83-94), and
// samples the next id from its last column; there is no max_seq stop (the window slides).
// Greedy runs entirely on the device (sh_window_greedy_decode); a sampled decode evaluates the
// window on the device (sh_prefill_logits, the EvalLogits forward) and draws on the host.
DecodeResult decode_window(sh_model *m, const sh_config &c, const std::vector<int32_t> &prompt_in, int seq,
                           int max_new, float temperature, Sampler &rng) {
    DecodeResult r;
    if (max_new <= 0) max_new = 64;
    if (temperature < 0) temperature = 0;
    auto account = [&]() {
        sh_timing t{};
        if (sh_stats(m, &t) == 0) {
            r.gpu_ms += t.gpu_ms;
            r.bytes += t.bytes_per_forward_mean * (double)t.forwards;
        }
    };
    std::vector<int32_t> prompt = prompt_in.empty() ? std::vector<int32_t>{1} : prompt_in;
    if ((int)prompt.size() > seq) prompt.erase(prompt.begin(), prompt.end() - seq);
    for (size_t i = 0; i < prompt.size(); i++)   // decode.go:44-48
        if (prompt[i] < 0 || prompt[i] >= c.vocab)
            fatalf("decode: %s", "storiesane decode: prompt token[" + std::to_string(i) + "]=" +
                                     std::to_string(prompt[i]) + " out of range");
    r.prompt_length = (int)prompt.size();
    if (temperature <= 1e-6f) {
        std::vector<int32_t> out(prompt.size() + max_new);
        int32_t n = 0, eos = 0;
        if (sh_window_greedy_decode(m, prompt.data(), (int32_t)prompt.size(), seq, max_new, out.data(), &n, &eos))
            fatalf("decode: %s", lib_error());
        account();
        r.tokens.assign(out.begin(), out.begin() + n);
        r.stopped_eos = eos != 0;
        return r;
    }
    r.tokens = prompt;
    std::vector<uint16_t> window(seq);
    std::vector<float> logits((size_t)c.vocab * seq), row(c.vocab);
    for (int step = 0; step < max_new; step++) {
        const size_t n = r.tokens.size(), keep = std::min(n, (size_t)seq);
        std::fill(window.begin(), window.end(), (uint16_t)1);
        for (size_t i = 0; i < keep; i++) window[seq - keep + i] = (uint16_t)r.tokens[n - keep + i];
        if (sh_prefill_logits(m, window.data(), seq, logits.data())) fatalf("decode: %s", lib_error());
        account();
        for (int v = 0; v < c.vocab; v++) row[v] = logits[(size_t)v * seq + seq - 1];
        const int next = rng.sample(row.data(), c.vocab, temperature);
        r.tokens.push_back(next);
        if (next == 2) {
            r.stopped_eos = true;
            break;
        }
    }
    return r;
}

}  // namespace

int main(int argc, char **argv) {
    Flags fl;
    fl.def("model", "");
    fl.def("ckpt", "");
    fl.def("tokenizer", "");
    fl.def("prompt-ids", "1");
    fl.def("max-new", "64");
    fl.def("temperature", "0.8");
    const std::string now = std::to_string(
        (long long)std::chrono::system_clock::now().time_since_epoch().count());
    fl.def("seed", now.c_str());
    fl.def("seq", "256");
    fl.def("ane", "false", true);
    fl.def("shape", "stories110m");
    fl.def("dtype", "");
    fl.def("kv", "");
    fl.def("synthetic-seed", "0");
    fl.def("synthetic-std", "0.02");
    fl.def("prompt-len", "0");
    fl.def("prompt-seed", "1");
    fl.def("bench-steps", "0");
    fl.def("bench-warmup", "2");
    fl.def("inspect", "false", true);
    fl.def("detokenize", "");
    fl.def("copy-calibrate", "0");
    fl.def("read-calibrate", "0");
    fl.def("batch", "0");
    fl.def("eval-logits", "false", true);
    fl.def("layers", "0");
    fl.def("train", "false", true);
    fl.def("lr", "3e-4");
    fl.parse(argc, argv);

    if (!fl.s("detokenize").empty()) {
        stories::Tokenizer tok;
        std::string err;
        const int vocab = fl.s("shape") == "qwen3-0.6b" ? 151936 : 32000;
        if (fl.s("tokenizer").empty()) fatalf("%s", "-detokenize needs -tokenizer");
        if (!tok.load(fl.s("tokenizer"), vocab, &err)) fatalf("load tokenizer: %s", err);
        std::string text;
        for (int32_t id : parse_token_list(fl.s("detokenize"))) text += tok.decode(id);
        printf("text=%s\n", text.c_str());
        return 0;
    }


    // ---- model description and host weights ----
    sh_config c{};
    stories::HostWeights w;
    std::string source;
    const std::string shape = fl.s("shape");
    if (!fl.s("ckpt").empty()) {   // main.go:113-122: a checkpoint overrides -model
        std::string err;
        stories::BlztMeta meta{};
        if (!stories::load_blzt_checkpoint(fl.s("ckpt"), &meta, &w, &err)) fatalf("decode: %s", err);
        if (fl.b("inspect")) {
            printf("%s\n", stories::describe_blzt_json(meta, w).c_str());
            return 0;
        }
        stories::config_from_blzt(meta, &c);
        source = "checkpoint";
    } else if (!fl.s("model").empty() && fl.s("model") != "synthetic") {
        std::string err;
        stories::Llama2Header hdr{};
        if (!stories::load_llama2_file(fl.s("model"), &hdr, &w, &err)) fatalf("decode: %s", err);
        if (fl.b("inspect")) {
            printf("%s\n", stories::describe_json(hdr, w).c_str());
            return 0;
        }
        stories::config_from_header(hdr, &c);
        source = "pretrained";
    } else {
        if (fl.b("inspect")) fatalf("%s", "-inspect needs -model");
        if (shape == "qwen3-0.6b") sh_config_qwen3_06b(&c);
        else if (shape == "stories110m") sh_config_stories110m(&c);
        else fatalf("unknown -shape %s", shape);
        source = "synthetic";
        if (fl.i("layers") > 0) c.n_layers = (int32_t)fl.i("layers");
    }
    // infer.go:84-89: maxSeq <= 0 -> 256, clamped to 256 for the Stories decoder
    long long seq = fl.i("seq");
    if (seq <= 0) seq = 256;
    if (shape == "stories110m" && seq > 256) seq = 256;
    c.max_seq = (int32_t)seq;
    int dtype = shape == "qwen3-0.6b" ? SH_DTYPE_BF16 : SH_DTYPE_F16;
    if (fl.s("dtype") == "fp16") dtype = SH_DTYPE_F16;
    else if (fl.s("dtype") == "bf16") dtype = SH_DTYPE_BF16;
    else if (fl.s("dtype") == "w8a8") dtype = SH_DTYPE_W8A8;
    else if (!fl.s("dtype").empty()) fatalf("unknown -dtype %s", fl.s("dtype"));
    if (fl.s("kv") == "f32") c.kv_dtype = SH_KV_F32;
    else if (fl.s("kv") == "f16") c.kv_dtype = SH_KV_F16;
    else if (fl.s("kv") == "bf16") c.kv_dtype = SH_KV_BF16;
    else if (!fl.s("kv").empty()) fatalf("unknown -kv %s", fl.s("kv"));
    if (source == "synthetic")
        synth_weights(c, (uint64_t)fl.i("synthetic-seed"), (float)fl.f("synthetic-std"), w);
    const int batch = (int)fl.i("batch");
    if (batch > 0) {
        if (fl.i("bench-steps") <= 0 || fl.i("prompt-len") <= 0)
            fatalf("%s", "-batch needs -bench-steps and -prompt-len");
        c.max_batch = batch;
    }
    const bool ane = fl.b("ane");
    if (ane) {
        // main.go:71-85: storiesane.Open with Seq = -seq; the engine scales each residual
        // branch by 1/sqrt(2 L) (residual.go:9)
        if (fl.i("bench-steps") > 0 || fl.i("batch") > 0 || fl.b("eval-logits") || fl.b("train"))
            fatalf("%s", "-ane takes no bench, batch, eval-logits or train flags");
        c.residual_scale = (float)(1.0 / sqrt(2.0 * c.n_layers));
    }
    if (fl.b("eval-logits")) {
        if (fl.i("bench-steps") <= 0 || fl.i("prompt-len") <= 0)
            fatalf("%s", "-eval-logits needs -bench-steps and -prompt-len");
        // the storiesane engine scales each residual branch by 1/sqrt(2 L) (residual.go:9)
        if (shape == "stories110m") c.residual_scale = (float)(1.0 / sqrt(2.0 * c.n_layers));
    }

    std::vector<int32_t> prompt;
    if (fl.i("prompt-len") > 0) {
        prompt.resize(fl.i("prompt-len"));
        if (sh_synth_tokens(prompt.data(), prompt.size(), (uint64_t)fl.i("prompt-seed"), c.vocab))
            fatalf("prompt: %s", lib_error());
    } else {
        prompt = parse_token_list(fl.s("prompt-ids"));
    }
    stories::Tokenizer tok;
    const bool have_tok = !fl.s("tokenizer").empty();
    if (have_tok) {
        std::string err;
        if (!tok.load(fl.s("tokenizer"), c.vocab, &err)) fatalf("load tokenizer: %s", err);
    }

    if (sh_init(0)) fatalf("decode: %s", lib_error());
    if (fl.b("train")) {
        // Engine.Step timing (engine.go:295-361): W untimed + K timed steps over drand48
        // windows of a synthetic token stream. FLOPs per step: the forward's, dX's and dW's
        // products (6 per weight per token), plus attention over the full S x S square per
        // head (forward QK^T and P.V, backward four products of the same size).
        const int steps = (int)fl.i("bench-steps");
        if (steps <= 0) fatalf("%s", "-train needs -bench-steps");
        sh_train_options o{};
        o.seq = (int32_t)c.max_seq;
        o.lr = (float)fl.f("lr");
        o.seed = fl.i("seed") ? fl.i("seed") : 42;
        c.residual_scale = (float)(1.0 / sqrt(2.0 * c.n_layers));   // residual.go:9
        sh_trainer *tr = sh_trainer_create(&c, &o);
        if (!tr) fatalf("train: %s", lib_error());
        for (int l = 0; l < c.n_layers; l++) {
            const stories::HostLayer &L = w.layers[l];
            if (sh_trainer_upload_layer(tr, l, L.wq.data(), L.wk.data(), L.wv.data(), L.wo.data(), L.w1.data(),
                                        L.w2.data(), L.w3.data(), L.rms_att.data(), L.rms_ffn.data()))
                fatalf("train: %s", lib_error());
        }
        if (sh_trainer_upload_globals(tr, w.embed.data(), w.rms_final.data())) fatalf("train: %s", lib_error());
        std::vector<int32_t> stream32(1 << 16);
        if (sh_synth_tokens(stream32.data(), stream32.size(), (uint64_t)fl.i("prompt-seed"), c.vocab))
            fatalf("train: %s", lib_error());
        std::vector<uint16_t> stream(stream32.begin(), stream32.end());
        if (sh_trainer_set_tokens(tr, stream.data(), (int64_t)stream.size())) fatalf("train: %s", lib_error());
        float loss = 0;
        for (int i = 0; i < fl.i("bench-warmup"); i++)
            if (sh_trainer_step(tr, &loss)) fatalf("train: %s", lib_error());
        std::vector<double> ms;
        std::vector<float> losses;
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; i++) {
            if (sh_trainer_step(tr, &loss)) fatalf("train: %s", lib_error());
            sh_train_state st{};
            sh_trainer_state(tr, &st);
            ms.push_back(st.last_step_ms);
            losses.push_back(loss);
        }
        const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        const double S = o.seq, D = c.dim, F = c.hidden;
        const double flops = 6.0 * S * (c.n_layers * (4.0 * D * D + 3.0 * D * F) + (double)c.vocab * D) +
                             12.0 * c.n_layers * S * S * D;
        std::string js = "{\"seq\": " + std::to_string(o.seq) + ", \"steps\": " + std::to_string(steps) +
                         ", \"warmup\": " + std::to_string(fl.i("bench-warmup")) + ", \"wall_s\": " +
                         std::to_string(wall) + ", \"step_ms\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(ms[i]);
        js += "], \"loss\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(losses[i]);
        char b[64];
        snprintf(b, sizeof b, "%.6e", flops);
        js += "], \"flops\": " + std::string(b) + "}";
        printf("%s\n", js.c_str());
        fflush(stdout);
        sh_trainer_destroy(tr);
        return 0;
    }
    sh_model *m = open_model(c, dtype, w);
    w = stories::HostWeights();   // device holds the weights now
    // the engine's decode seeds its generator with -seed, or 42 when that is 0
    // (decode.go:30-33, engine.go:166-168)
    Sampler rng{(uint64_t)(ane && fl.i("seed") == 0 ? 42 : fl.i("seed"))};
    const int max_new = (int)fl.i("max-new");
    const float temperature = (float)fl.f("temperature");

    const int steps = (int)fl.i("bench-steps");
    // Any bench mode may first time the library's plain copy kernel: a known byte count for
    // scaling the profiler's traffic counters, and the achievable HBM bandwidth.
    double copy_ms = 0, copy_gbs = 0;
    const long long copy_bytes = steps > 0 ? fl.i("copy-calibrate") : 0;
    if (copy_bytes > 0 && sh_copy_calibrate((size_t)copy_bytes, 5, &copy_ms, &copy_gbs))
        fatalf("copy calibrate: %s", lib_error());
    double read_ms = 0, read_gbs = 0;
    const long long read_bytes = steps > 0 ? fl.i("read-calibrate") : 0;
    if (read_bytes > 0 && sh_read_calibrate((size_t)read_bytes, 5, &read_ms, &read_gbs))
        fatalf("read calibrate: %s", lib_error());
    if (steps > 0 && batch > 0) {
        // Batched greedy decode timing: B prompts of prompt-len ids, max-new steps each.
        const int plen = (int)fl.i("prompt-len");
        std::vector<int32_t> prompts((size_t)batch * plen);
        if (sh_synth_tokens(prompts.data(), prompts.size(), (uint64_t)fl.i("prompt-seed"), c.vocab))
            fatalf("prompts: %s", lib_error());
        const int stride = plen + (max_new > 0 ? max_new : 64);
        std::vector<int32_t> out((size_t)batch * stride), n_out(batch);
        auto run = [&]() {
            if (sh_batch_greedy_decode(m, prompts.data(), batch, plen, max_new, out.data(), n_out.data()))
                fatalf("batch decode: %s", lib_error());
        };
        for (int i = 0; i < fl.i("bench-warmup"); i++) run();
        std::vector<double> dec_ms, pre_ms;
        std::vector<long long> fwd, gen;
        double bytes = 0;
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; i++) {
            run();
            sh_timing t{};
            if (sh_stats(m, &t)) fatalf("stats: %s", lib_error());
            dec_ms.push_back(t.gpu_ms);
            pre_ms.push_back(t.prefill_ms);
            fwd.push_back(t.forwards);
            gen.push_back(t.tokens_out);
            bytes = t.bytes_per_forward_mean;
        }
        const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        std::string js = "{\"batch\": " + std::to_string(batch) + ", \"prompt_len\": " + std::to_string(plen) +
                         ", \"steps\": " + std::to_string(steps) + ", \"wall_s\": " + std::to_string(wall) +
                         ", \"decode_ms\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(dec_ms[i]);
        js += "], \"prefill_ms\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(pre_ms[i]);
        js += "], \"decode_steps\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(fwd[i]);
        js += "], \"tokens_out\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(gen[i]);
        char b[64];
        snprintf(b, sizeof b, "%.1f", bytes);
        js += "], \"bytes_per_step_mean\": " + std::string(b) + ", \"copy_gbs\": " + std::to_string(copy_gbs) +
              ", \"read_gbs\": " + std::to_string(read_gbs) + ", \"tokens_row0\": [" +
              join_ints(std::vector<int32_t>(out.begin(), out.begin() + n_out[0])) + "]}";
        printf("%s\n", js.c_str());
        fflush(stdout);
        sh_model_destroy(m);
        return 0;
    }
    if (steps > 0 && fl.b("eval-logits")) {
        // Full-sequence forward timing: W untimed, then K timed EvalLogits calls over the
        // prompt. FLOPs: 2 per weight per row for every projection and the classifier, and
        // the attention's QK^T and P.V over the full S x S square per head (the count the
        // reference's channel-first forward performs).
        const int S = (int)prompt.size();
        if (S > c.max_seq) fatalf("%s", "-prompt-len exceeds -seq (" + std::to_string(c.max_seq) + ")");
        std::vector<uint16_t> ids(prompt.begin(), prompt.end());
        std::vector<float> logits((size_t)c.vocab * S);
        auto run = [&]() {
            if (sh_prefill_logits(m, ids.data(), S, logits.data()))
                fatalf("eval logits: %s", lib_error());
        };
        for (int i = 0; i < fl.i("bench-warmup"); i++) run();
        std::vector<double> gpu_ms;
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; i++) {
            run();
            sh_timing t{};
            if (sh_stats(m, &t)) fatalf("stats: %s", lib_error());
            gpu_ms.push_back(t.gpu_ms);
        }
        const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        const double qdim = (double)c.n_heads * c.head_dim, kvdim = (double)c.n_kv_heads * c.head_dim;
        const double per_layer = (double)c.dim * (qdim + 2 * kvdim) + qdim * c.dim + 3.0 * c.dim * c.hidden;
        const double params = per_layer * c.n_layers + (double)c.vocab * c.dim;
        const double flops = 2.0 * S * params + 4.0 * c.n_layers * c.n_heads * (double)S * S * c.head_dim;
        double sum = 0;
        for (float v : logits) sum += v;
        char b[160];
        snprintf(b, sizeof b, "], \"flops\": %.6e, \"logits_sum\": %.6e}", flops, sum);
        std::string js = "{\"seq\": " + std::to_string(S) + ", \"steps\": " + std::to_string(steps) +
                         ", \"warmup\": " + std::to_string(fl.i("bench-warmup")) +
                         ", \"wall_s\": " + std::to_string(wall) + ", \"gpu_ms\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(gpu_ms[i]);
        js += b;
        printf("%s\n", js.c_str());
        fflush(stdout);
        sh_model_destroy(m);
        return 0;
    }
    if (steps > 0) {
        // Greedy decode timing for bench harnesses: W untimed runs, then K timed ones.
        for (int i = 0; i < fl.i("bench-warmup"); i++) decode(m, c, prompt, max_new, 0.f, rng);
        std::vector<double> gpu_ms, bytes, pre_ms;
        std::vector<long long> fwd, gen;
        DecodeResult last;
        int persistent = 0, grid = 0;
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < steps; i++) {
            last = decode(m, c, prompt, max_new, 0.f, rng);
            sh_timing t{};
            if (sh_stats(m, &t)) fatalf("stats: %s", lib_error());
            gpu_ms.push_back(t.gpu_ms);
            pre_ms.push_back(t.prefill_ms);
            fwd.push_back(t.forwards);
            gen.push_back(t.tokens_out);
            bytes.push_back(t.bytes_per_forward_mean);
            persistent = t.persistent;
            grid = t.grid;
        }
        const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        char desc[1024];
        sh_model_describe(m, desc, sizeof desc);
        std::string js = "{\"steps\": " + std::to_string(steps) +
                         ", \"warmup\": " + std::to_string(fl.i("bench-warmup")) +
                         ", \"wall_s\": " + std::to_string(wall) + ", \"gpu_ms\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(gpu_ms[i]);
        js += "], \"prefill_ms\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(pre_ms[i]);
        js += "], \"forwards\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(fwd[i]);
        js += "], \"generated\": [";
        for (int i = 0; i < steps; i++) js += (i ? ", " : "") + std::to_string(gen[i]);
        js += "], \"bytes_per_forward_mean\": [";
        for (int i = 0; i < steps; i++) {
            char b[64];
            snprintf(b, sizeof b, "%.1f", bytes[i]);
            js += (i ? ", " : "") + std::string(b);
        }
        js += "], \"persistent\": " + std::to_string(persistent) +
              ", \"grid\": " + std::to_string(grid) +
              ", \"copy_bytes\": " + std::to_string(copy_bytes) +
              ", \"copy_gbs\": " + std::to_string(copy_gbs) +
              ", \"read_gbs\": " + std::to_string(read_gbs) +
              ", \"prompt_length\": " + std::to_string(last.prompt_length) +
              ", \"tokens\": [" + join_ints(last.tokens) + "]" +
              ", \"describe\": \"" + json_escape(desc) + "\"}";
        printf("%s\n", js.c_str());
        fflush(stdout);
        sh_model_destroy(m);
        return 0;
    }

    const auto t0 = std::chrono::steady_clock::now();
    DecodeResult res = ane ? decode_window(m, c, prompt, (int)c.max_seq, max_new, temperature, rng)
                           : decode(m, c, prompt, max_new, temperature, rng);
    const double elapsed = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    const int new_tokens = (int)res.tokens.size() - res.prompt_length;
    const double tps = elapsed > 0 ? new_tokens / elapsed : 0.0;
    // main.go:60-67's line, plus the device-side rate: algorithmic bytes of the forwards
    // (weights, norms, KV rows, logits) over their device time, and its fraction of the
    // 8 TB/s HBM peak
    const double hbm_gbps = res.gpu_ms > 0 ? res.bytes / (res.gpu_ms * 1e6) : 0.0;
    printf("source=%s prompt_tokens=%d generated_tokens=%d elapsed=%s tok/s=%.2f eos=%s "
           "hbm_gbps=%.1f roofline_frac=%.4f\n",
           source.c_str(), res.prompt_length, new_tokens, go_duration(elapsed).c_str(), tps,
           res.stopped_eos ? "true" : "false", hbm_gbps, hbm_gbps / 8000.0);
    printf("tokens=%s\n", join_ints(res.tokens).c_str());
    if (have_tok) {
        std::string text;
        for (size_t i = res.prompt_length; i < res.tokens.size(); i++) text += tok.decode(res.tokens[i]);
        printf("text=%s\n", text.c_str());
    } else {
        printf("text=(tokenizer not provided)\n");
    }
    sh_model_destroy(m);
    return 0;
}
