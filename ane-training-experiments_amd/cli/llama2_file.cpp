// llama2_file.cpp — see llama2_file.hpp.
#include "llama2_file.hpp"

#include <errno.h>
#include <stdio.h>
#include <string.h>

namespace stories {

namespace {

bool read_f32s(FILE *f, std::vector<float> &dst, const std::string &what, std::string *err) {
    if (dst.empty()) return true;
    const size_t got = fread(dst.data(), sizeof(float), dst.size(), f);
    if (got != dst.size()) {
        *err = "read " + what + ": unexpected EOF";
        return false;
    }
    return true;
}

double sum(const std::vector<float> &v) {
    double s = 0;
    for (float x : v) s += (double)x;
    return s;
}

}  // namespace

void HostWeights::resize(const sh_config &c) {
    const size_t D = c.dim, F = c.hidden, Q = (size_t)c.n_heads * c.head_dim,
                 KV = (size_t)c.n_kv_heads * c.head_dim;
    layers.assign(c.n_layers, HostLayer());
    for (HostLayer &L : layers) {
        L.wq.assign(Q * D, 0.f);
        L.wk.assign(KV * D, 0.f);
        L.wv.assign(KV * D, 0.f);
        L.wo.assign(D * Q, 0.f);
        L.w1.assign(F * D, 0.f);
        L.w2.assign(D * F, 0.f);
        L.w3.assign(F * D, 0.f);
        L.rms_att.assign(D, 1.f);
        L.rms_ffn.assign(D, 1.f);
        L.q_norm.assign(c.qk_norm ? c.head_dim : 0, 1.f);
        L.k_norm.assign(c.qk_norm ? c.head_dim : 0, 1.f);
    }
    embed.assign((size_t)c.vocab * D, 0.f);
    rms_final.assign(D, 1.f);
    cls.assign(c.tied_embed ? 0 : (size_t)c.vocab * D, 0.f);
    shared_classifier = c.tied_embed != 0;
}

void config_from_header(const Llama2Header &h, sh_config *c) {
    memset(c, 0, sizeof *c);
    c->dim = h.dim;
    c->hidden = h.hidden;
    c->n_layers = h.n_layers;
    c->n_heads = h.n_heads;
    c->n_kv_heads = h.n_kv_heads;
    c->head_dim = h.dim / h.n_heads;
    c->vocab = h.vocab < 0 ? -h.vocab : h.vocab;
    c->max_seq = h.seq_len;
    c->rope_theta = 10000.0;
    c->norm_eps = 1e-5;
    c->qk_norm_eps = 1e-6;
    c->residual_scale = 1.0f;
    c->qk_norm = 0;
    c->tied_embed = 1;
    c->kv_dtype = SH_KV_F32;
    c->max_batch = 1;
}

bool load_llama2_file(const std::string &path, Llama2Header *hdr, HostWeights *w, std::string *err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        *err = "open " + path + ": " + strerror(errno);
        return false;
    }
    bool ok = fread(hdr, sizeof *hdr, 1, f) == 1;
    if (!ok) *err = "read config: unexpected EOF";
    if (ok && (hdr->dim <= 0 || hdr->hidden <= 0 || hdr->n_layers <= 0 || hdr->n_heads <= 0 ||
               hdr->n_kv_heads <= 0 || hdr->vocab == 0 || hdr->dim % hdr->n_heads ||
               hdr->n_heads % hdr->n_kv_heads)) {
        char b[256];
        snprintf(b, sizeof b, "config mismatch: got dim=%d hidden=%d layers=%d heads=%d kv_heads=%d vocab=%d",
                 hdr->dim, hdr->hidden, hdr->n_layers, hdr->n_heads, hdr->n_kv_heads, hdr->vocab);
        *err = b;
        ok = false;
    }
    if (!ok) {
        fclose(f);
        return false;
    }
    sh_config c;
    config_from_header(*hdr, &c);
    w->resize(c);
    w->shared_classifier = hdr->vocab > 0;
    const int L = hdr->n_layers;
    ok = read_f32s(f, w->embed, "embed", err);
    struct Field {
        const char *name;
        std::vector<float> HostLayer::*member;
    };
    const Field fields[] = {{"rms_att", &HostLayer::rms_att}, {"wq", &HostLayer::wq},
                            {"wk", &HostLayer::wk},           {"wv", &HostLayer::wv},
                            {"wo", &HostLayer::wo},           {"rms_ffn", &HostLayer::rms_ffn},
                            {"w1", &HostLayer::w1},           {"w2", &HostLayer::w2},
                            {"w3", &HostLayer::w3}};
    for (const Field &fd : fields)
        for (int l = 0; ok && l < L; l++)
            ok = read_f32s(f, w->layers[l].*fd.member, std::string(fd.name) + "[" + std::to_string(l) + "]", err);
    ok = ok && read_f32s(f, w->rms_final, "rms_final", err);
    fclose(f);
    return ok;
}

std::string describe_json(const Llama2Header &h, const HostWeights &w) {
    char b[512];
    snprintf(b, sizeof b,
             "{\"header\": {\"dim\": %d, \"hidden\": %d, \"n_layers\": %d, \"n_heads\": %d, "
             "\"n_kv_heads\": %d, \"vocab\": %d, \"seq_len\": %d}, \"shared_classifier\": %s, \"sums\": {",
             h.dim, h.hidden, h.n_layers, h.n_heads, h.n_kv_heads, h.vocab, h.seq_len,
             w.shared_classifier ? "true" : "false");
    std::string s = b;
    auto add = [&](const char *name, double v, bool last) {
        char t[128];
        snprintf(t, sizeof t, "\"%s\": %.17g%s", name, v, last ? "" : ", ");
        s += t;
    };
    add("embed", sum(w.embed), false);
    const char *names[] = {"rms_att", "wq", "wk", "wv", "wo", "rms_ffn", "w1", "w2", "w3"};
    std::vector<float> HostLayer::*members[] = {&HostLayer::rms_att, &HostLayer::wq, &HostLayer::wk,
                                                &HostLayer::wv,      &HostLayer::wo, &HostLayer::rms_ffn,
                                                &HostLayer::w1,      &HostLayer::w2, &HostLayer::w3};
    for (int k = 0; k < 9; k++) {
        double t = 0;
        for (const HostLayer &L : w.layers) t += sum(L.*members[k]);
        add(names[k], t, false);
    }
    add("rms_final", sum(w.rms_final), true);
    s += "}}";
    return s;
}

bool Tokenizer::load(const std::string &path, int vocab, std::string *err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        *err = "open " + path + ": " + strerror(errno);
        return false;
    }
    int32_t max_len = 0;
    bool ok = fread(&max_len, 4, 1, f) == 1;
    if (!ok) *err = "read tokenizer header: unexpected EOF";
    if (ok && max_len <= 0) {
        *err = "bad tokenizer header: max token len=" + std::to_string(max_len);
        ok = false;
    }
    vocab_.assign(ok ? vocab : 0, std::string());
    for (int i = 0; ok && i < vocab; i++) {
        float score;
        int32_t n;
        if (fread(&score, 4, 1, f) != 1) {
            *err = "unexpected EOF at token " + std::to_string(i);
            ok = false;
        } else if (fread(&n, 4, 1, f) != 1) {
            *err = "read token[" + std::to_string(i) + "] length: unexpected EOF";
            ok = false;
        } else if (n < 0 || (int64_t)n > (int64_t)max_len * 8) {
            *err = "bad token[" + std::to_string(i) + "] length=" + std::to_string(n);
            ok = false;
        } else {
            vocab_[i].resize(n);
            if (n && fread(&vocab_[i][0], 1, n, f) != (size_t)n) {
                *err = "read token[" + std::to_string(i) + "] bytes: unexpected EOF";
                ok = false;
            }
        }
    }
    fclose(f);
    return ok;
}

static int hex_nibble(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

std::string Tokenizer::decode(int id) const {
    if (id < 0 || id >= (int)vocab_.size()) return "";
    const std::string &s = vocab_[id];
    if (s.size() >= 5 && s.compare(0, 3, "<0x") == 0 && s.back() == '>') {
        if (s.size() == 6) {
            const int hi = hex_nibble(s[3]), lo = hex_nibble(s[4]);
            if (hi >= 0 && lo >= 0) return std::string(1, (char)((hi << 4) | lo));
        }
    }
    return s;
}

}  // namespace stories
