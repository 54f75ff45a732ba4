// llama2_file.hpp — host-side readers for the llama2.c model and tokenizer files that
// ane/stories reads (weights.go:49-122 LoadPretrained, tokenizer.go:16-97 LoadTokenizer).
// Plain C++; no device code.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "stories_hip.h"

namespace stories {

// weights.go / config.go:20-28 Llama2Config: seven little-endian int32 at offset 0.
struct Llama2Header {
    int32_t dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len;
};

// One layer in the reference's row-major [out, in] layout (weights.go:13-17).
struct HostLayer {
    std::vector<float> wq, wk, wv, wo, w1, w2, w3, rms_att, rms_ffn, q_norm, k_norm;
};

struct HostWeights {
    std::vector<HostLayer> layers;
    std::vector<float> embed, rms_final, cls;   // cls empty when tied
    bool shared_classifier = true;              // weights.go:68 SharedCL = vocab > 0
    void resize(const sh_config &c);            // sizes every tensor for c; gains = 1
};

// LoadPretrained order: embed, rms_att[L], wq[L], wk[L], wv[L], wo[L], rms_ffn[L], w1[L],
// w2[L], w3[L], rms_final. wk/wv hold n_kv_heads * (dim / n_heads) rows each. Any classifier
// stored after rms_final is not read: the reference decoder projects with Embed
// (infer.go:242) whatever SharedCL says. Errors name the tensor, like the reference.
bool load_llama2_file(const std::string &path, Llama2Header *hdr, HostWeights *w, std::string *err);

// sh_config for a file header: head_dim = dim / n_heads, theta 10000, eps 1e-5, alpha 1,
// tied classifier, fp32 KV cache (infer.go:97-113), max_seq = seq_len.
void config_from_header(const Llama2Header &h, sh_config *c);

// {"header": {...}, "sums": {"embed": s, "wq": s, ...}} with float64 sums over all layers.
std::string describe_json(const Llama2Header &h, const HostWeights &w);

// Training checkpoint header and meta (ane/stories/ckpt.go:237-447, magic "BLZT",
// versions 2 and 3).
struct BlztMeta {
    int32_t version, step, total_steps, n_layers, vocab, dim, hidden, heads, seq;
    float lr, loss;
    double cum_compile, cum_train, cum_wall;
    int32_t cum_steps, cum_batches, adam_t;
};

// loadCheckpointFile (ckpt.go:249-447) without optimizer state: the header, then per layer
// Wq, Wk, Wv, Wo, W1, W2, W3, RMSAtt, RMSFFN, then every layer's Adam moments (skipped),
// RMSFinal and its moments (skipped), Embed and its moments (skipped). The reference accepts
// only the Stories110M constants; here the shapes come from the header (wq/wk/wv/wo are
// dim x dim, w1/w3 hidden x dim, w2 dim x hidden, as that format has no grouped heads), so
// small checkpoints of the same layout load too. Errors follow the reference's wording.
bool load_blzt_checkpoint(const std::string &path, BlztMeta *meta, HostWeights *w, std::string *err);
void config_from_blzt(const BlztMeta &h, sh_config *c);
std::string describe_blzt_json(const BlztMeta &h, const HostWeights &w);

// tokenizer.go:16-97.
class Tokenizer {
  public:
    bool load(const std::string &path, int vocab, std::string *err);
    // Decode: "" for ids out of range; "<0xHH>" pieces become the byte HH.
    std::string decode(int id) const;

  private:
    std::vector<std::string> vocab_;
};

}  // namespace stories
