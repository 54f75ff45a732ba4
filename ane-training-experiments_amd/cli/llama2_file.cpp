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

void config_from_blzt(const BlztMeta &h, sh_config *c) {
    Llama2Header l{h.dim, h.hidden, h.n_layers, h.heads, h.heads, h.vocab, h.seq};
    config_from_header(l, c);
}

bool load_blzt_checkpoint(const std::string &path, BlztMeta *meta, HostWeights *w, std::string *err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        *err = "open " + path + ": " + strerror(errno);
        return false;
    }
    bool ok = true;
    auto rd = [&](void *dst, size_t n) {
        if (ok && fread(dst, 1, n, f) != n) {
            *err = "unexpected EOF";
            ok = false;
        }
    };
    int32_t magic = 0;
    BlztMeta &m = *meta;
    memset(&m, 0, sizeof m);
    rd(&magic, 4);
    rd(&m.version, 4);
    if (ok && (magic != 0x424C5A54 || (m.version != 2 && m.version != 3))) {   // ckpt.go:279-281
        char b[96];
        snprintf(b, sizeof b, "bad checkpoint header magic=%x version=%d", (unsigned)magic, m.version);
        *err = b;
        ok = false;
    }
    rd(&m.step, 4);
    rd(&m.total_steps, 4);
    rd(&m.n_layers, 4);
    rd(&m.vocab, 4);
    rd(&m.dim, 4);
    rd(&m.hidden, 4);
    rd(&m.heads, 4);
    rd(&m.seq, 4);
    if (ok && (m.n_layers <= 0 || m.vocab <= 0 || m.dim <= 0 || m.hidden <= 0 || m.heads <= 0 ||
               m.dim % m.heads)) {
        *err = "checkpoint config mismatch";
        ok = false;
    }
    rd(&m.lr, 4);
    rd(&m.loss, 4);
    rd(&m.cum_compile, 8);
    rd(&m.cum_train, 8);
    rd(&m.cum_wall, 8);
    rd(&m.cum_steps, 4);
    rd(&m.cum_batches, 4);
    rd(&m.adam_t, 4);
    int32_t reserved[3];
    rd(reserved, 12);
    if (!ok) {
        fclose(f);
        return false;
    }
    sh_config c;
    config_from_blzt(m, &c);
    w->resize(c);
    const char *names[] = {"wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn"};
    std::vector<float> HostLayer::*members[] = {&HostLayer::wq, &HostLayer::wk, &HostLayer::wv,
                                                &HostLayer::wo, &HostLayer::w1, &HostLayer::w2,
                                                &HostLayer::w3, &HostLayer::rms_att,
                                                &HostLayer::rms_ffn};
    size_t layer_floats = 0;
    for (int l = 0; ok && l < m.n_layers; l++)
        for (int k = 0; ok && k < 9; k++) {
            std::vector<float> &v = w->layers[l].*members[k];
            ok = read_f32s(f, v, std::string(names[k]) + "[" + std::to_string(l) + "]", err);
            if (l == 0) layer_floats += v.size();
        }
    // every layer's Adam moments (M and V of the nine tensors), then RMSFinal
    auto skip = [&](size_t floats) {
        if (ok && fseek(f, (long)(floats * 4), SEEK_CUR) != 0) {
            *err = "skip optimizer state: seek failed";
            ok = false;
        }
    };
    skip(2 * layer_floats * (size_t)m.n_layers);
    ok = ok && read_f32s(f, w->rms_final, "rms_final", err);
    skip(2 * (size_t)m.dim);
    ok = ok && read_f32s(f, w->embed, "embed", err);
    // the file must hold Embed's moments too: a short file fails as the reference's read would
    if (ok) {
        const long here = ftell(f);
        fseek(f, 0, SEEK_END);
        const long end = ftell(f);
        if (end - here < (long)(2 * w->embed.size() * 4)) {
            *err = "read embed optimizer state: unexpected EOF";
            ok = false;
        }
    }
    fclose(f);
    return ok;
}

std::string describe_blzt_json(const BlztMeta &h, const HostWeights &w) {
    char b[640];
    snprintf(b, sizeof b,
             "{\"checkpoint\": {\"version\": %d, \"step\": %d, \"total_steps\": %d, "
             "\"n_layers\": %d, \"vocab\": %d, \"dim\": %d, \"hidden\": %d, \"heads\": %d, "
             "\"seq\": %d, \"lr\": %.9g, \"loss\": %.9g, \"cum_compile\": %.17g, "
             "\"cum_train\": %.17g, \"cum_wall\": %.17g, \"cum_steps\": %d, \"cum_batches\": %d, "
             "\"adam_t\": %d}, ",
             h.version, h.step, h.total_steps, h.n_layers, h.vocab, h.dim, h.hidden, h.heads, h.seq,
             h.lr, h.loss, h.cum_compile, h.cum_train, h.cum_wall, h.cum_steps, h.cum_batches,
             h.adam_t);
    Llama2Header l{h.dim, h.hidden, h.n_layers, h.heads, h.heads, h.vocab, h.seq};
    std::string s = describe_json(l, w);
    return std::string(b) + s.substr(1);   // merge the two objects
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
