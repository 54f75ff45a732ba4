// sh_api.hip — the C ABI declared in include/stories_hip.h: model lifetime, weight upload,
// the device-resident decode loop (one captured HIP graph per token forward), and the
// device quantizer entry points.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "sh_internal.hpp"

namespace sh {

static thread_local std::string g_err;
static thread_local int g_device = 0;

void set_error(const std::string &msg) { g_err = msg; }

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return false;
}

bool gemv_supported(int cols, bool pairs);

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t weight_elem_bytes(int dtype) { return dtype == SH_DTYPE_W8A8 ? 1 : 2; }
size_t kv_elem_bytes(int kv) { return kv == SH_KV_F32 ? 4 : 2; }

bool valid_config(const sh_config &c, int dtype) {
    auto fail = [](const std::string &m) {
        set_error("invalid config: " + m);
        return false;
    };
    if (dtype != SH_DTYPE_F16 && dtype != SH_DTYPE_BF16 && dtype != SH_DTYPE_W8A8)
        return fail("dtype must be SH_DTYPE_F16, SH_DTYPE_BF16 or SH_DTYPE_W8A8");
    if (c.dim <= 0 || c.hidden <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
        c.vocab <= 0 || c.max_seq <= 0)
        return fail("sizes must be positive");
    if (c.n_heads % c.n_kv_heads) return fail("n_heads must be a multiple of n_kv_heads");
    if (c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256)
        return fail("head_dim must be 32, 64, 128 or 256");
    if (c.max_seq > kMaxSeqLds) return fail("max_seq above 4096");
    if (c.kv_dtype < SH_KV_F32 || c.kv_dtype > SH_KV_BF16) return fail("kv_dtype");
    if (c.max_batch < 1) return fail("max_batch must be >= 1");
    const int qdim = c.n_heads * c.head_dim;
    if (!gemv_supported(c.dim, true)) return fail("dim has no GEMV tiling");
    if (!gemv_supported(qdim, false)) return fail("n_heads*head_dim has no GEMV tiling");
    if (!gemv_supported(c.hidden, false)) return fail("hidden has no GEMV tiling");
    return true;
}

struct HostBuf {
    std::vector<uint8_t> v;
};

// Algorithmic bytes of one forward at position pos: every weight byte once, norms, the
// K/V rows 0..pos read, one K/V row written, the embedding row and the logits written.
double forward_bytes(const sh_model *m, int pos) {
    const sh_config &c = m->cfg;
    const double eb = (double)weight_elem_bytes(m->dtype);
    const double D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim;
    double per_layer = eb * ((Q + 2 * KV) * D + D * Q + 2 * F * D + D * F) + 4.0 * 2 * D;
    if (m->dtype == SH_DTYPE_W8A8) per_layer += 4.0 * ((Q + 2 * KV) + D + 2 * F + D);  // row scales
    if (c.qk_norm) per_layer += 4.0 * 2 * c.head_dim;
    const double kvb = (double)kv_elem_bytes(c.kv_dtype);
    per_layer += kvb * 2 * KV * (double)(pos + 1);  // K and V rows read
    per_layer += kvb * 2 * KV;                        // K and V row written
    double total = per_layer * c.n_layers;
    total += eb * (double)c.vocab * D + 4.0 * D;      // classifier rows + final norm
    if (m->dtype == SH_DTYPE_W8A8) total += 4.0 * c.vocab;   // classifier row scales
    total += 2.0 * D;                                 // embedding row
    total += 4.0 * c.vocab;                           // logits written
    return total;
}

// Compulsory HBM bytes of one full-sequence forward: every weight once, the embedding rows,
// the logits written. Activations of a few MB stay in the 256 MB of L2 + MALL.
double prefill_bytes(const sh_model *m, int S) {
    const sh_config &c = m->cfg;
    const double eb = (double)weight_elem_bytes(m->dtype);
    const double D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim;
    double per_layer = eb * ((Q + 2 * KV) * D + D * Q + 2 * F * D + D * F) + 4.0 * 2 * D;
    return per_layer * c.n_layers + eb * (double)c.vocab * D + eb * D * S + 4.0 * c.vocab * S;
}

hipError_t ensure_step_graph(sh_model *m) {
    if (m->step_ready) return hipSuccess;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return e;
    hipError_t e2 = enqueue_decode_step(m);
    e = hipStreamEndCapture(m->stream, &g);
    if (e2 != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return e2;
    }
    if (e != hipSuccess) return e;
    e = hipGraphInstantiate(&m->step_exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return e;
    m->step_ready = true;
    return hipSuccess;
}

// Hand-over words of a stage's output vector (padded producer blocks), of the gate vector
// and of the argmax partials (two forwards' slots per workgroup).
size_t stage_words(const sh_model *m, int st) { return (size_t)m->p_own[st].n * (size_t)m->p_ostride[st]; }
size_t gate_words(const sh_model *m) { return stage_words(m, 2); }
size_t arg_words(const sh_model *m) { return 2 * (size_t)m->p_grid * kArgSlot; }

// Runs n_forwards forwards from pos0 with the persistent kernel (epochs advance; the
// hand-over buffers are cleared before the 32-bit epoch space runs out).
bool run_persistent(sh_model *m, int pos0, int n_forwards, int n_prompt) {
    const uint64_t need = (uint64_t)n_forwards * (uint64_t)(m->cfg.n_layers + 1);
    if ((uint64_t)m->epoch + need >= 0xF0000000ull) {
        struct {
            uint64_t *p;
            size_t n;
        } ll[] = {{m->ll_qkv, (size_t)m->qkv_rows}, {m->ll_att, (size_t)m->qdim},
                  {m->ll_x2, stage_words(m, 1)},    {m->ll_gate, gate_words(m)},
                  {m->ll_x, stage_words(m, 3)},     {m->ll_pv, arg_words(m)},
                  {m->ll_pi, arg_words(m)}};
        for (auto &b : ll)
            if (!hip_ok(hipMemsetAsync(b.p, 0, 8 * b.n, m->stream), "clear hand-over")) return false;
        m->epoch = 1;
    }
    if (!hip_ok(hipMemsetAsync(m->p_err, 0, 8, m->stream), "clear err")) return false;
    return hip_ok(launch_persistent(m, pos0, n_forwards, n_prompt), "persistent decode launch");
}

// Outcome of a persistent launch, read after the stream has synchronised.
enum class LaunchCheck { Ok, Absent, Failed };

// Ok: the launch ran to its end. Absent: a wait expired before every workgroup had started
// (the grid was not all resident, e.g. another process held CUs). Failed: the error word could
// not be read, or a wait expired with every workgroup running (a hand-over that never came:
// reported, never retried).
LaunchCheck check_persistent_err(sh_model *m) {
    int err = 0;
    if (!hip_ok(hipMemcpy(&err, m->p_err, 4, hipMemcpyDeviceToHost), "read err")) return LaunchCheck::Failed;
    if (err == 0) return LaunchCheck::Ok;
    if (err == kErrAbsent) {
        set_error("persistent decode: a hand-over wait expired before every workgroup had started "
                  "(the grid was not all resident)");
        return LaunchCheck::Absent;
    }
    set_error("persistent decode: a hand-over wait exceeded its time bound with every workgroup running");
    return LaunchCheck::Failed;
}

// After a persistent launch whose grid was not all resident: models with a per-stage path
// switch to it for good and the caller repeats the call (which starts from a cleared cache or,
// for one forward, rewrites the cache row it evaluates); W8A8 has no per-stage path and keeps
// the error.
bool fall_back_to_graph(sh_model *m) {
    if (m->dtype == SH_DTYPE_W8A8) return false;
    m->persistent = false;
    snprintf(m->path_note, sizeof(m->path_note), "%s",
             "per-stage kernels in a HIP graph (a persistent decode launch timed out waiting "
             "for its workgroups to be resident)");
    return true;
}

// The outcome of the persistent launch a call just waited for: true to carry on, false to
// return -1; *retry is set when the model has switched to the per-stage path and the call
// should run again.
bool persistent_outcome(sh_model *m, bool *retry) {
    *retry = false;
    if (!m->persistent) return true;
    switch (check_persistent_err(m)) {
    case LaunchCheck::Ok: return true;
    case LaunchCheck::Absent:
        if (!fall_back_to_graph(m)) return false;
        *retry = true;
        return true;
    default: return false;
    }
}

// Enqueues n forwards at positions pos0.. (tokens[pos] feeds each; from n_prompt on the
// argmax is appended): one persistent launch, or one graph replay per forward.
bool launch_forwards(sh_model *m, int pos0, int n, int n_prompt) {
    if (m->persistent) return run_persistent(m, pos0, n, n_prompt);
    if (!hip_ok(ensure_step_graph(m), "capture decode step")) return false;
    DecodeState st{};
    st.pos = pos0;
    st.n_prompt = n_prompt;
    if (!hip_ok(hipMemcpyAsync(m->state, &st, sizeof(st), hipMemcpyHostToDevice, m->stream), "state"))
        return false;
    for (int f = 0; f < n; f++)
        if (!hip_ok(hipGraphLaunch(m->step_exec, m->stream), "hipGraphLaunch")) return false;
    return true;
}

bool ready(const sh_model *m) {
    if (!m) {
        set_error("nil model");
        return false;
    }
    if (m->uploaded_layers != m->cfg.n_layers || !m->globals_uploaded) {
        set_error("model weights are not fully uploaded");
        return false;
    }
    return true;
}

uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <typename F>
void parallel_ranges(size_t n, F fn) {
    unsigned hw = std::thread::hardware_concurrency();
    unsigned nt = std::max(1u, std::min(hw ? hw : 1u, 16u));
    if (n < (1u << 16)) nt = 1;
    std::vector<std::thread> th;
    const size_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        const size_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        th.emplace_back([=] { fn(a, b); });
    }
    for (auto &t : th) t.join();
}

// Shared set-up of the channel-first seams: checks, prefill scratch for seq rows, the rows'
// positions 0..seq-1 of one sequence, and x_cf [dim, seq] copied into pf_cf.
bool seam_begin(sh_model *m, const char *what, const float *x_cf, int32_t seq, void *out,
                bool logits, bool need_globals) {
    if (!m) {
        set_error("nil model");
        return false;
    }
    // the layer seam needs only the layers (a one-layer model per compiled layer, as
    // compileStoriesLayerForwardFunc makes them); the final norm and classifier the globals
    if (m->uploaded_layers != m->cfg.n_layers || (need_globals && !m->globals_uploaded)) {
        set_error(std::string(what) + ": model weights are not fully uploaded");
        return false;
    }
    if (!x_cf || !out || seq <= 0 || seq > m->cfg.max_seq) {
        set_error(std::string(what) + ": bad arguments");
        return false;
    }
    std::string why;
    if (!prefill_supported(m, &why)) {
        set_error(std::string(what) + ": " + why);
        return false;
    }
    (void)hipSetDevice(m->device);
    if (!hip_ok(prefill_alloc(m, seq, logits), "prefill scratch")) return false;
    std::vector<int32_t> rows(2 * (size_t)seq);
    for (int t = 0; t < seq; t++) {
        rows[t] = t;
        rows[(size_t)seq + t] = 0;
    }
    const size_t xb = sizeof(float) * (size_t)m->cfg.dim * seq;
    return hip_ok(hipMemcpyAsync(m->pf_rowpos, rows.data(), 4 * (size_t)seq, hipMemcpyHostToDevice, m->stream), "seam rows") &&
           hip_ok(hipMemcpyAsync(m->pf_rowseq, rows.data() + seq, 4 * (size_t)seq, hipMemcpyHostToDevice, m->stream), "seam rows") &&
           hip_ok(hipMemcpyAsync(m->pf_cf, x_cf, xb, hipMemcpyHostToDevice, m->stream), "seam input") &&
           hip_ok(hipEventRecord(m->ev0, m->stream), "event");
}

// Copies `bytes` of device results to the host, waits, and records the device time.
bool seam_end(sh_model *m, const void *dev, void *host, size_t bytes, int seq) {
    if (!hip_ok(hipEventRecord(m->ev1, m->stream), "event") ||
        !hip_ok(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, m->stream), "seam output") ||
        !hip_ok(hipStreamSynchronize(m->stream), "seam sync"))
        return false;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, m->ev0, m->ev1);
    m->last = sh_timing{};
    m->last.gpu_ms = ms;
    m->last.forwards = 1;
    m->last.tokens_out = seq;
    return true;
}

uint16_t host_bf16_bits(float x);

// Device scratch of the allocation-free entry point (sh_conv_eval_noalloc): the operand
// planes of its input and the K-range partials of its product. One copy per GPU, resident
// until the process ends. In host code `scratch` names a host-side stand-in, never the
// device memory: the device address comes from hipGetSymbolAddress with that device current
// (at sh_init, or at the entry point's first call on a device) and is kept per device.
constexpr size_t kNoAllocScratchBytes = 16u << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on `device`, which must be the current device; NULL (and
// the error text set) if the runtime cannot resolve it.
void *scratch_address(int device) {
    if (device < 0 || device >= kMaxDevices) {
        set_error("device index beyond the no-alloc scratch table");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return nullptr;
        g_scratch_ptr[device] = p;
    }
    return g_scratch_ptr[device];
}

}  // namespace
}  // namespace sh

using namespace sh;

extern "C" {

int sh_init(int32_t device) {
    int n = 0;
    if (!hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount")) return -1;
    if (device < 0 || device >= n) {
        set_error("sh_init: device " + std::to_string(device) + " out of range");
        return -1;
    }
    if (!hip_ok(hipSetDevice(device), "hipSetDevice")) return -1;
    g_device = device;
    // resolve this device's no-alloc scratch now, outside any caller's capture or loop
    return scratch_address(device) ? 0 : -1;
}

size_t sh_last_error(char *buf, size_t len) {
    if (buf && len) {
        const size_t n = std::min(len - 1, g_err.size());
        memcpy(buf, g_err.data(), n);
        buf[n] = 0;
    }
    return g_err.size();
}

int sh_config_stories110m(sh_config *c) {
    if (!c) return -1;
    memset(c, 0, sizeof(*c));
    c->dim = 768;
    c->hidden = 2048;
    c->n_layers = 12;
    c->n_heads = 12;
    c->n_kv_heads = 12;
    c->head_dim = 64;
    c->vocab = 32000;
    c->max_seq = 256;
    c->rope_theta = 10000.0;
    c->norm_eps = 1e-5;
    c->qk_norm_eps = 1e-6;
    c->residual_scale = 1.0f;
    c->qk_norm = 0;
    c->tied_embed = 1;
    c->kv_dtype = SH_KV_F32;
    c->max_batch = 1;
    return 0;
}

int sh_config_qwen3_06b(sh_config *c) {
    if (!c) return -1;
    memset(c, 0, sizeof(*c));
    c->dim = 1024;
    c->hidden = 3072;
    c->n_layers = 28;
    c->n_heads = 16;
    c->n_kv_heads = 8;
    c->head_dim = 128;
    c->vocab = 151936;
    c->max_seq = 2048;
    c->rope_theta = 1000000.0;
    c->norm_eps = 1e-6;
    c->qk_norm_eps = 1e-6;
    c->residual_scale = 1.0f;
    c->qk_norm = 1;
    c->tied_embed = 1;
    c->kv_dtype = SH_KV_BF16;
    c->max_batch = 1;
    return 0;
}

sh_model *sh_model_create(const sh_config *cfg, int32_t dtype) {
    if (!cfg) {
        set_error("sh_model_create: nil config");
        return nullptr;
    }
    if (!valid_config(*cfg, dtype)) return nullptr;
    if (!hip_ok(hipSetDevice(g_device), "hipSetDevice")) return nullptr;
    if (!hip_ok(gemm_setup(), "GEMM set-up")) return nullptr;
    sh_model *m = new sh_model();
    memset((void *)m, 0, sizeof(*m));
    m->cfg = *cfg;
    m->dtype = dtype;
    m->device = g_device;
    const sh_config &c = m->cfg;
    m->qdim = c.n_heads * c.head_dim;
    m->kvdim = c.n_kv_heads * c.head_dim;
    m->qkv_rows = m->qdim + 2 * m->kvdim;
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    const size_t eb = weight_elem_bytes(dtype);
    const bool w8 = dtype == SH_DTYPE_W8A8;

    // weight arena layout
    std::vector<size_t> offs;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    struct LOff {
        size_t wqkv, wo, w13, w2, sqkv, so, s13, s2, ra, rf, qn, kn;
    };
    std::vector<LOff> lo(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        lo[l].wqkv = take(eb * m->qkv_rows * D);
        lo[l].wo = take(eb * D * m->qdim);
        lo[l].w13 = take(eb * 2 * F * D);
        lo[l].w2 = take(eb * D * F);
        lo[l].sqkv = w8 ? take(4 * m->qkv_rows) : 0;
        lo[l].so = w8 ? take(4 * D) : 0;
        lo[l].s13 = w8 ? take(4 * 2 * F) : 0;
        lo[l].s2 = w8 ? take(4 * D) : 0;
        lo[l].ra = take(4 * D);
        lo[l].rf = take(4 * D);
        lo[l].qn = c.qk_norm ? take(4 * c.head_dim) : 0;
        lo[l].kn = c.qk_norm ? take(4 * c.head_dim) : 0;
    }
    const size_t o_embed = take(2 * V * D);
    const bool own_cls = !c.tied_embed || w8;
    const size_t o_cls = own_cls ? take(eb * V * D) : 0;
    const size_t o_scls = w8 ? take(4 * V) : 0;
    const size_t o_rmsf = take(4 * D);
    m->arena_bytes = off;

    auto fail = [&](const char *what, hipError_t e) -> sh_model * {
        hip_ok(e, what);
        sh_model_destroy(m);
        return nullptr;
    };
    hipError_t e;
    if ((e = hipMalloc(&m->arena, m->arena_bytes)) != hipSuccess) return fail("hipMalloc arena", e);
    uint8_t *A = (uint8_t *)m->arena;
    m->layers = new LayerDev[c.n_layers];
    for (int l = 0; l < c.n_layers; l++) {
        LayerDev &L = m->layers[l];
        L.wqkv = A + lo[l].wqkv;
        L.wo = A + lo[l].wo;
        L.w13 = A + lo[l].w13;
        L.w2 = A + lo[l].w2;
        L.s_qkv = w8 ? (float *)(A + lo[l].sqkv) : nullptr;
        L.s_o = w8 ? (float *)(A + lo[l].so) : nullptr;
        L.s_13 = w8 ? (float *)(A + lo[l].s13) : nullptr;
        L.s_2 = w8 ? (float *)(A + lo[l].s2) : nullptr;
        L.rms_att = (float *)(A + lo[l].ra);
        L.rms_ffn = (float *)(A + lo[l].rf);
        L.q_norm = c.qk_norm ? (float *)(A + lo[l].qn) : nullptr;
        L.k_norm = c.qk_norm ? (float *)(A + lo[l].kn) : nullptr;
    }
    m->embed = A + o_embed;
    m->cls = own_cls ? (void *)(A + o_cls) : m->embed;
    m->s_cls = w8 ? (float *)(A + o_scls) : nullptr;
    m->rms_final = (float *)(A + o_rmsf);

    m->kv_elems = (size_t)c.max_batch * c.n_layers * c.max_seq * m->kvdim;
    const size_t kvb = kv_elem_bytes(c.kv_dtype) * m->kv_elems;
    if ((e = hipMalloc(&m->kcache, kvb)) != hipSuccess) return fail("hipMalloc kcache", e);
    if ((e = hipMalloc(&m->vcache, kvb)) != hipSuccess) return fail("hipMalloc vcache", e);

    // RoPE tables, infer.go:97-107: float64 angle, float32 cos/sin
    const int half = c.head_dim / 2;
    std::vector<float> rc((size_t)c.max_seq * half), rs((size_t)c.max_seq * half);
    for (int pos = 0; pos < c.max_seq; pos++)
        for (int i = 0; i < half; i++) {
            const double freq =
                (double)pos / pow(c.rope_theta, (double)(2 * i) / (double)c.head_dim);
            rc[(size_t)pos * half + i] = (float)cos(freq);
            rs[(size_t)pos * half + i] = (float)sin(freq);
        }
    if ((e = hipMalloc(&m->rope_cos, rc.size() * 4)) != hipSuccess) return fail("hipMalloc rope", e);
    if ((e = hipMalloc(&m->rope_sin, rs.size() * 4)) != hipSuccess) return fail("hipMalloc rope", e);
    if ((e = hipMemcpy(m->rope_cos, rc.data(), rc.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
        return fail("hipMemcpy rope", e);
    if ((e = hipMemcpy(m->rope_sin, rs.data(), rs.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
        return fail("hipMemcpy rope", e);

    const size_t widest = std::max({D, (size_t)m->qkv_rows, 2 * F, (size_t)m->qdim});
    m->n_partials = gemv_partials(m);
    if (m->n_partials <= 0) return fail("classifier tiling", hipErrorInvalidValue);
    if ((e = hipMalloc(&m->x, 4 * D)) != hipSuccess) return fail("hipMalloc x", e);
    if ((e = hipMalloc(&m->x2, 4 * D)) != hipSuccess) return fail("hipMalloc x2", e);
    if ((e = hipMalloc(&m->qkv, 4 * widest)) != hipSuccess) return fail("hipMalloc qkv", e);
    if ((e = hipMalloc(&m->att, 4 * widest)) != hipSuccess) return fail("hipMalloc att", e);
    if ((e = hipMalloc(&m->gate, 4 * F)) != hipSuccess) return fail("hipMalloc gate", e);
    if ((e = hipMalloc(&m->logits, 4 * V)) != hipSuccess) return fail("hipMalloc logits", e);
    if ((e = hipMalloc(&m->partials, sizeof(ArgmaxPartial) * m->n_partials)) != hipSuccess)
        return fail("hipMalloc partials", e);
    if ((e = hipMalloc(&m->tokens, 4 * (c.max_seq + 1))) != hipSuccess) return fail("hipMalloc tokens", e);
    if ((e = hipMalloc(&m->argmax_hist, 4 * (c.max_seq + 1))) != hipSuccess)
        return fail("hipMalloc hist", e);
    if ((e = hipMalloc(&m->state, sizeof(DecodeState))) != hipSuccess) return fail("hipMalloc state", e);
    if ((e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking)) != hipSuccess)
        return fail("hipStreamCreate", e);
    if ((e = hipEventCreate(&m->ev0)) != hipSuccess) return fail("hipEventCreate", e);
    if ((e = hipEventCreate(&m->ev1)) != hipSuccess) return fail("hipEventCreate", e);
    if ((e = hipEventCreate(&m->ev_mid)) != hipSuccess) return fail("hipEventCreate", e);
    if ((e = hipMemsetAsync(m->kcache, 0, kvb, m->stream)) != hipSuccess) return fail("memset kv", e);
    if ((e = hipMemsetAsync(m->vcache, 0, kvb, m->stream)) != hipSuccess) return fail("memset kv", e);
    if ((e = hipMemsetAsync(m->tokens, 0, 4 * (c.max_seq + 1), m->stream)) != hipSuccess)
        return fail("memset tokens", e);
    if ((e = hipStreamSynchronize(m->stream)) != hipSuccess) return fail("sync", e);

    // persistent decode kernel: chosen when the shape has an instantiation and fits the CUs
    {
        std::string why;
        hipError_t ge = hipSuccess;
        if (!persistent_supported(m)) {
            why = "shape/dtype has no persistent-kernel instantiation";
        } else if ((ge = persistent_plan(m, &why)) == hipSuccess) {
            m->persistent = true;
        } else {
            why += std::string("; grid: ") + hipGetErrorString(ge);
        }
        const std::string note =
            m->persistent ? "persistent decode kernel, grid " + std::to_string(m->p_grid) + " (" + why + ")"
                          : "per-stage kernels in a HIP graph (" + why + ")";
        snprintf(m->path_note, sizeof(m->path_note), "%s", note.c_str());
        if (w8 && !m->persistent) {
            // the per-stage kernels have no int8 GEMV; W8A8 runs only in the persistent kernel
            set_error("invalid config: W8A8 decode needs a persistent-kernel shape (" + why + ")");
            sh_model_destroy(m);
            return nullptr;
        }
    }
    if (m->persistent) {
        const size_t lpb = persistent_layer_ptr_bytes(c.n_layers);
        std::vector<uint8_t> lp(lpb);
        persistent_fill_layer_ptrs(m, lp.data());
        if ((e = hipMalloc(&m->p_layers, lpb)) != hipSuccess) return fail("hipMalloc layer ptrs", e);
        if ((e = hipMemcpy(m->p_layers, lp.data(), lpb, hipMemcpyHostToDevice)) != hipSuccess)
            return fail("upload layer ptrs", e);
        struct {
            uint64_t **p;
            size_t n;
        } ll[] = {{&m->ll_qkv, (size_t)m->qkv_rows}, {&m->ll_att, (size_t)m->qdim},
                  {&m->ll_x2, stage_words(m, 1)},    {&m->ll_gate, gate_words(m)},
                  {&m->ll_x, stage_words(m, 3)},     {&m->ll_pv, arg_words(m)},
                  {&m->ll_pi, arg_words(m)}};
        for (auto &b : ll) {
            if ((e = hipMalloc(b.p, 8 * b.n)) != hipSuccess) return fail("hipMalloc hand-over", e);
            if ((e = hipMemset(*b.p, 0, 8 * b.n)) != hipSuccess) return fail("clear hand-over", e);
        }
        if ((e = hipMalloc(&m->p_err, 64)) != hipSuccess) return fail("hipMalloc err", e);
        if ((e = hipMemset(m->p_err, 0, 64)) != hipSuccess) return fail("clear err", e);
        int rate_khz = 0;
        if ((e = hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, m->device)) != hipSuccess)
            return fail("wall clock rate", e);
        m->spin_ticks = (long long)(rate_khz > 0 ? rate_khz : 100000) * 1000LL * 2;  // 2 s
        m->epoch = 1;  // cleared words carry epoch 0
        const size_t tb = (size_t)m->p_grid * 2 * (5 * (size_t)c.n_layers + 3) * sizeof(long long);
        if ((e = hipMalloc(&m->trace_buf, tb)) != hipSuccess) return fail("hipMalloc trace", e);
        if ((e = hipMemset(m->trace_buf, 0, tb)) != hipSuccess) return fail("clear trace", e);
    }
    m->trace_f = -1;
    return m;
}

void sh_model_destroy(sh_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->step_ready) (void)hipGraphExecDestroy(m->step_exec);
    (void)hipFree(m->arena);
    (void)hipFree(m->kcache);
    (void)hipFree(m->vcache);
    (void)hipFree(m->rope_cos);
    (void)hipFree(m->rope_sin);
    (void)hipFree(m->x);
    (void)hipFree(m->x2);
    (void)hipFree(m->qkv);
    (void)hipFree(m->att);
    (void)hipFree(m->gate);
    (void)hipFree(m->logits);
    (void)hipFree(m->partials);
    (void)hipFree(m->tokens);
    (void)hipFree(m->argmax_hist);
    (void)hipFree(m->state);
    (void)hipFree(m->p_layers);
    (void)hipFree(m->ll_qkv);
    (void)hipFree(m->ll_att);
    (void)hipFree(m->ll_x2);
    (void)hipFree(m->ll_gate);
    (void)hipFree(m->ll_x);
    (void)hipFree(m->ll_pv);
    (void)hipFree(m->ll_pi);
    (void)hipFree(m->p_err);
    (void)hipFree(m->trace_buf);
    (void)hipFree(m->pf_arena);
    (void)hipFree(m->tap_buf);
    if (m->bt_ready) (void)hipGraphExecDestroy(m->bt_exec);
    (void)hipFree(m->bt_arena);
    if (m->wd_ready) (void)hipGraphExecDestroy(m->wd_exec);
    if (m->pf_ready) (void)hipGraphExecDestroy(m->pf_exec);
    (void)hipFree(m->wd_arena);
    if (m->ev0) (void)hipEventDestroy(m->ev0);
    if (m->ev1) (void)hipEventDestroy(m->ev1);
    if (m->ev_mid) (void)hipEventDestroy(m->ev_mid);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete[] m->layers;
    delete m;
}

static int upload_matrix(sh_model *m, float *staging, const float *host, int rows, int cols,
                         void *dst, float *scales, int stride, int offset) {
    const size_t n = (size_t)rows * cols;
    if (!hip_ok(hipMemcpyAsync(staging, host, n * 4, hipMemcpyHostToDevice, m->stream),
                "upload weights"))
        return -1;
    hipError_t e;
    if (m->dtype == SH_DTYPE_W8A8)
        e = launch_quantize_rows(staging, (int8_t *)dst, scales, rows, cols, stride, offset, stride,
                                 offset, m->stream);
    else
        e = launch_convert_rows(staging, dst, rows, cols, m->dtype, stride, offset, m->stream);
    if (!hip_ok(e, "convert weights")) return -1;
    // staging is reused by the next matrix
    return hip_ok(hipStreamSynchronize(m->stream), "upload sync") ? 0 : -1;
}

int sh_model_upload_layer(sh_model *m, int32_t layer, const float *wq, const float *wk,
                          const float *wv, const float *wo, const float *w1, const float *w2,
                          const float *w3, const float *rms_att, const float *rms_ffn,
                          const float *q_norm, const float *k_norm) {
    if (!m) {
        set_error("sh_model_upload_layer: nil model");
        return -1;
    }
    const sh_config &c = m->cfg;
    if (layer < 0 || layer >= c.n_layers) {
        set_error("sh_model_upload_layer: layer out of range");
        return -1;
    }
    if (!wq || !wk || !wv || !wo || !w1 || !w2 || !w3 || !rms_att || !rms_ffn ||
        (c.qk_norm && (!q_norm || !k_norm))) {
        set_error("sh_model_upload_layer: missing tensor");
        return -1;
    }
    (void)hipSetDevice(m->device);
    const int D = c.dim, F = c.hidden;
    const size_t biggest = std::max({(size_t)m->qdim * D, (size_t)F * D});
    float *staging = nullptr;
    if (!hip_ok(hipMalloc(&staging, biggest * 4), "hipMalloc staging")) return -1;
    LayerDev &L = m->layers[layer];
    const size_t eb = weight_elem_bytes(m->dtype);
    int rc = 0;
    rc |= upload_matrix(m, staging, wq, m->qdim, D, L.wqkv, L.s_qkv, 1, 0);
    rc |= upload_matrix(m, staging, wk, m->kvdim, D, L.wqkv, L.s_qkv, 1, m->qdim);
    rc |= upload_matrix(m, staging, wv, m->kvdim, D, L.wqkv, L.s_qkv, 1, m->qdim + m->kvdim);
    rc |= upload_matrix(m, staging, wo, D, m->qdim, L.wo, L.s_o, 1, 0);
    rc |= upload_matrix(m, staging, w1, F, D, L.w13, L.s_13, 2, 0);
    rc |= upload_matrix(m, staging, w3, F, D, L.w13, L.s_13, 2, 1);
    rc |= upload_matrix(m, staging, w2, D, F, L.w2, L.s_2, 1, 0);
    (void)eb;
    (void)hipFree(staging);
    if (rc) return -1;
    if (!hip_ok(hipMemcpy(L.rms_att, rms_att, 4 * D, hipMemcpyHostToDevice), "upload rms_att") ||
        !hip_ok(hipMemcpy(L.rms_ffn, rms_ffn, 4 * D, hipMemcpyHostToDevice), "upload rms_ffn"))
        return -1;
    if (c.qk_norm &&
        (!hip_ok(hipMemcpy(L.q_norm, q_norm, 4 * c.head_dim, hipMemcpyHostToDevice), "upload q_norm") ||
         !hip_ok(hipMemcpy(L.k_norm, k_norm, 4 * c.head_dim, hipMemcpyHostToDevice), "upload k_norm")))
        return -1;
    m->uploaded_layers = std::min(m->uploaded_layers + 1, c.n_layers);
    return 0;
}

int sh_model_upload_globals(sh_model *m, const float *embed, const float *rms_final,
                            const float *cls) {
    if (!m) {
        set_error("sh_model_upload_globals: nil model");
        return -1;
    }
    const sh_config &c = m->cfg;
    if (!embed || !rms_final || (!c.tied_embed && !cls)) {
        set_error("sh_model_upload_globals: missing tensor");
        return -1;
    }
    (void)hipSetDevice(m->device);
    const size_t n = (size_t)c.vocab * c.dim;
    float *staging = nullptr;
    if (!hip_ok(hipMalloc(&staging, n * 4), "hipMalloc staging")) return -1;
    int rc = 0;
    // the lookup table: fp16 for F16 and W8A8, bf16 for BF16
    const int lookup_dtype = m->dtype == SH_DTYPE_BF16 ? SH_DTYPE_BF16 : SH_DTYPE_F16;
    if (!hip_ok(hipMemcpy(staging, embed, n * 4, hipMemcpyHostToDevice), "upload embed")) rc = -1;
    if (!rc && !hip_ok(launch_convert_rows(staging, m->embed, c.vocab, c.dim, lookup_dtype, 1, 0,
                                           m->stream), "convert embed"))
        rc = -1;
    if (!rc && !hip_ok(hipStreamSynchronize(m->stream), "sync")) rc = -1;
    if (!rc && m->cls != m->embed) {
        const float *src = c.tied_embed ? embed : cls;
        rc = upload_matrix(m, staging, src, c.vocab, c.dim, m->cls, m->s_cls, 1, 0);
    }
    (void)hipFree(staging);
    if (rc) return -1;
    if (!hip_ok(hipMemcpy(m->rms_final, rms_final, 4 * c.dim, hipMemcpyHostToDevice), "upload rms_final"))
        return -1;
    m->globals_uploaded = true;
    return 0;
}

int sh_model_read_weights(const sh_model *m, int32_t layer, const char *name, void *dst, size_t bytes) {
    if (!m || !name || !dst) {
        set_error("sh_model_read_weights: bad arguments");
        return -1;
    }
    const sh_config &c = m->cfg;
    const bool w8 = m->dtype == SH_DTYPE_W8A8;
    const size_t eb = weight_elem_bytes(m->dtype);
    std::string n(name);
    const bool scale = n.size() > 6 && n.compare(n.size() - 6, 6, ".scale") == 0;
    if (scale) n.resize(n.size() - 6);
    if (scale && !w8) {
        set_error("sh_model_read_weights: row scales exist only for W8A8 models");
        return -1;
    }
    // the tensor as rows [r0, r0 + rows) of a matrix whose row r lives at row r*step + r0 of
    // its storage (w1 and w3 are interleaved in w13)
    const void *base = nullptr;
    const float *sbase = nullptr;
    int rows = 0, cols = 0, r0 = 0, step = 1;
    size_t elem = eb;
    if (layer >= 0) {
        if (layer >= c.n_layers) {
            set_error("sh_model_read_weights: layer out of range");
            return -1;
        }
        const LayerDev &L = m->layers[layer];
        if (n == "wq") { base = L.wqkv; sbase = L.s_qkv; rows = m->qdim; cols = c.dim; }
        else if (n == "wk") { base = L.wqkv; sbase = L.s_qkv; rows = m->kvdim; cols = c.dim; r0 = m->qdim; }
        else if (n == "wv") { base = L.wqkv; sbase = L.s_qkv; rows = m->kvdim; cols = c.dim; r0 = m->qdim + m->kvdim; }
        else if (n == "wo") { base = L.wo; sbase = L.s_o; rows = c.dim; cols = m->qdim; }
        else if (n == "w1") { base = L.w13; sbase = L.s_13; rows = c.hidden; cols = c.dim; step = 2; }
        else if (n == "w3") { base = L.w13; sbase = L.s_13; rows = c.hidden; cols = c.dim; step = 2; r0 = 1; }
        else if (n == "w2") { base = L.w2; sbase = L.s_2; rows = c.dim; cols = c.hidden; }
    } else if (layer == -1) {
        if (n == "embed" && !scale) {
            base = m->embed; rows = c.vocab; cols = c.dim; elem = 2;   // the 16-bit lookup table
        } else if (n == "cls" && (m->cls != m->embed || scale)) {
            base = m->cls; sbase = m->s_cls; rows = c.vocab; cols = c.dim;
        }
    }
    if (!base) {
        set_error(std::string("sh_model_read_weights: no tensor ") + name + " at layer " + std::to_string(layer));
        return -1;
    }
    const size_t row_bytes = scale ? 4 : (size_t)cols * elem;
    if (bytes != row_bytes * rows) {
        set_error("sh_model_read_weights: " + std::string(name) + " holds " + std::to_string(row_bytes * rows) +
                  " bytes");
        return -1;
    }
    (void)hipSetDevice(m->device);
    const uint8_t *src = scale ? (const uint8_t *)sbase : (const uint8_t *)base;
    return hip_ok(hipMemcpy2D(dst, row_bytes, src + (size_t)r0 * row_bytes, row_bytes * step, row_bytes, rows,
                              hipMemcpyDeviceToHost), "read weights") ? 0 : -1;
}

int sh_reset_cache(sh_model *m) {
    if (!m) {
        set_error("sh_reset_cache: nil model");
        return -1;
    }
    (void)hipSetDevice(m->device);
    const size_t kvb = kv_elem_bytes(m->cfg.kv_dtype) * m->kv_elems;
    if (!hip_ok(hipMemsetAsync(m->kcache, 0, kvb, m->stream), "reset kcache") ||
        !hip_ok(hipMemsetAsync(m->vcache, 0, kvb, m->stream), "reset vcache") ||
        !hip_ok(hipStreamSynchronize(m->stream), "reset sync"))
        return -1;
    return 0;
}

int sh_decode_step(sh_model *m, int32_t token, int32_t pos, float *logits, int32_t *argmax_out) {
    if (!ready(m)) return -1;
    const sh_config &c = m->cfg;
    if (token < 0 || token >= c.vocab) {
        set_error("token out of range: " + std::to_string(token));
        return -1;
    }
    if (pos < 0 || pos >= c.max_seq) {
        set_error("position out of range: " + std::to_string(pos));
        return -1;
    }
    (void)hipSetDevice(m->device);
    // never append: this call only evaluates
    if (!hip_ok(hipMemcpyAsync(m->tokens + pos, &token, 4, hipMemcpyHostToDevice, m->stream), "token") ||
        !hip_ok(hipEventRecord(m->ev0, m->stream), "event") || !launch_forwards(m, pos, 1, c.max_seq + 1) ||
        !hip_ok(hipEventRecord(m->ev1, m->stream), "event"))
        return -1;
    if (logits &&
        !hip_ok(hipMemcpyAsync(logits, m->logits, 4 * (size_t)c.vocab, hipMemcpyDeviceToHost, m->stream),
                "copy logits"))
        return -1;
    int32_t am = 0;
    if (!hip_ok(hipMemcpyAsync(&am, m->argmax_hist + pos, 4, hipMemcpyDeviceToHost, m->stream), "argmax") ||
        !hip_ok(hipStreamSynchronize(m->stream), "decode step"))
        return -1;
    bool retry = false;
    if (!persistent_outcome(m, &retry)) return -1;
    if (retry) return sh_decode_step(m, token, pos, logits, argmax_out);
    if (argmax_out) *argmax_out = am;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, m->ev0, m->ev1);
    m->last = sh_timing{};
    m->last.gpu_ms = ms;
    m->last.forwards = 1;
    m->last.tokens_out = 0;
    m->last.bytes_per_forward_mean = forward_bytes(m, pos);
    m->last.persistent = m->persistent ? 1 : 0;
    m->last.grid = m->persistent ? m->p_grid : 0;
    return 0;
}

int sh_greedy_decode(sh_model *m, const int32_t *prompt, int32_t n_prompt, int32_t max_new,
                     int32_t *out_tokens, int32_t *n_out, int32_t *stopped_eos) {
    if (!ready(m)) return -1;
    if (!out_tokens || !n_out || !stopped_eos) {
        set_error("sh_greedy_decode: nil output");
        return -1;
    }
    const sh_config &c = m->cfg;
    // infer.go:140-163: defaults, empty prompt -> [BOS], keep the last max_seq ids, validate
    if (max_new <= 0) max_new = 64;
    const int32_t bos = kBos;
    if (n_prompt <= 0 || !prompt) {
        prompt = &bos;
        n_prompt = 1;
    }
    if (n_prompt > c.max_seq) {
        prompt += n_prompt - c.max_seq;
        n_prompt = c.max_seq;
    }
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= c.vocab) {
            set_error("prompt token[" + std::to_string(i) + "]=" + std::to_string(prompt[i]) +
                      " out of range");
            return -1;
        }
    (void)hipSetDevice(m->device);
    // infer.go:179: generate while step < maxNew and len(tokens) < maxSeq
    const int generated = std::min(max_new, c.max_seq - n_prompt);
    const int forwards = n_prompt - 1 + generated;
    const size_t kvb = kv_elem_bytes(c.kv_dtype) * m->kv_elems;
    if (!hip_ok(hipMemcpyAsync(m->tokens, prompt, 4 * (size_t)n_prompt, hipMemcpyHostToDevice, m->stream),
                "prompt"))
        return -1;
    // The prompt's first n_prompt-1 positions only fill the KV cache (their logits are never
    // read): one causal forward over them on the full-sequence path, in the decode forms of
    // the softmax sum and SiLU, stores the cache a token-by-token decode would store, to the
    // rounding of its fp32 sums (W8A8: bit for bit, its full-sequence forward keeping the
    // decode's per-token quantization, float order and exact attention). The token loop then
    // starts at the last prompt id.
    std::string why;
    const int pre = (n_prompt > 1 && !m->no_prompt_prefill && prefill_supported(m, &why)) ? n_prompt - 1 : 0;
    if (pre > 0) {
        if (!hip_ok(prefill_alloc(m, pre, false), "prefill scratch")) return -1;
        std::vector<int32_t> rows(3 * (size_t)pre);
        for (int t = 0; t < pre; t++) {
            rows[t] = prompt[t];
            rows[pre + t] = t;
            rows[2 * (size_t)pre + t] = 0;
        }
        if (!hip_ok(hipMemcpyAsync(m->pf_tokens, rows.data(), 4 * (size_t)pre, hipMemcpyHostToDevice, m->stream), "prompt rows") ||
            !hip_ok(hipMemcpyAsync(m->pf_rowpos, rows.data() + pre, 4 * (size_t)pre, hipMemcpyHostToDevice, m->stream), "prompt rows") ||
            !hip_ok(hipMemcpyAsync(m->pf_rowseq, rows.data() + 2 * (size_t)pre, 4 * (size_t)pre, hipMemcpyHostToDevice, m->stream), "prompt rows"))
            return -1;
    }
    // timed region: cache reset (infer.go:165-168), the prompt forward, every token forward
    if (!hip_ok(hipEventRecord(m->ev0, m->stream), "event")) return -1;
    if (!hip_ok(hipMemsetAsync(m->kcache, 0, kvb, m->stream), "reset kcache") ||
        !hip_ok(hipMemsetAsync(m->vcache, 0, kvb, m->stream), "reset vcache"))
        return -1;
    if (pre > 0 && !hip_ok(enqueue_prefill(m, pre, pre, false, true), "prompt forward")) return -1;
    if (!hip_ok(hipEventRecord(m->ev_mid, m->stream), "event")) return -1;
    if (forwards > pre && !launch_forwards(m, pre, forwards - pre, n_prompt)) return -1;
    if (!hip_ok(hipEventRecord(m->ev1, m->stream), "event")) return -1;
    const int total = n_prompt + generated;
    if (!hip_ok(hipMemcpyAsync(out_tokens, m->tokens, 4 * (size_t)total, hipMemcpyDeviceToHost, m->stream),
                "copy tokens") ||
        !hip_ok(hipStreamSynchronize(m->stream), "greedy decode"))
        return -1;
    bool retry = false;
    if (!persistent_outcome(m, &retry)) return -1;
    if (retry) return sh_greedy_decode(m, prompt, n_prompt, max_new, out_tokens, n_out, stopped_eos);
    // infer.go:190-193: stop after EOS
    int n = n_prompt;
    int eos = 0;
    for (int i = n_prompt; i < total; i++) {
        n = i + 1;
        if (out_tokens[i] == kEos) {
            eos = 1;
            break;
        }
    }
    *n_out = n;
    *stopped_eos = eos;
    float ms = 0, pre_ms = 0;
    (void)hipEventElapsedTime(&ms, m->ev0, m->ev1);
    (void)hipEventElapsedTime(&pre_ms, m->ev0, m->ev_mid);
    double bytes = 0;
    for (int p = pre; p < forwards; p++) bytes += forward_bytes(m, p);
    m->last.gpu_ms = ms;
    m->last.forwards = forwards - pre;
    m->last.tokens_out = n - n_prompt;
    m->last.bytes_per_forward_mean = forwards > pre ? bytes / (forwards - pre) : 0;
    m->last.persistent = m->persistent ? 1 : 0;
    m->last.grid = m->persistent ? m->p_grid : 0;
    m->last.prefill_ms = pre_ms;
    return 0;
}

int sh_prefill_logits(sh_model *m, const uint16_t *tokens, int32_t seq, float *logits_cf) {
    if (!ready(m)) return -1;
    if (!tokens || !logits_cf || seq <= 0 || seq > m->cfg.max_seq) {
        set_error("sh_prefill_logits: bad arguments");
        return -1;
    }
    std::string why;
    if (!prefill_supported(m, &why)) {
        set_error("sh_prefill_logits: " + why);
        return -1;
    }
    (void)hipSetDevice(m->device);
    if (!hip_ok(prefill_alloc(m, seq, true), "prefill scratch")) return -1;
    // rows: the ids (out-of-range ones embed as zeros), positions 0..seq-1, one sequence
    std::vector<int32_t> rows(3 * (size_t)seq);
    for (int t = 0; t < seq; t++) {
        rows[t] = tokens[t];
        rows[seq + t] = t;
        rows[2 * (size_t)seq + t] = 0;
    }
    if (!hip_ok(hipMemcpyAsync(m->pf_tokens, rows.data(), 4 * (size_t)seq, hipMemcpyHostToDevice, m->stream), "prefill tokens") ||
        !hip_ok(hipMemcpyAsync(m->pf_rowpos, rows.data() + seq, 4 * (size_t)seq, hipMemcpyHostToDevice, m->stream), "prefill rows") ||
        !hip_ok(hipMemcpyAsync(m->pf_rowseq, rows.data() + 2 * (size_t)seq, 4 * (size_t)seq, hipMemcpyHostToDevice, m->stream), "prefill rows"))
        return -1;
    // the forward's ~110 kernels run as one captured graph, replayed while the length and
    // the scratch stay the same
    if (!m->pf_ready || m->pf_graph_seq != seq) {
        if (m->pf_ready) (void)hipGraphExecDestroy(m->pf_exec);
        m->pf_ready = false;
        hipGraph_t g = nullptr;
        if (!hip_ok(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal), "capture")) return -1;
        // EvalLogits, whose bar is the logits: the fp16 products take the activations as one
        // fp16 plane (an 11-bit significand); bf16 keeps the hi/lo pair, whose one plane would
        // carry 8 bits. Forwards that fill a decode cache keep the pair.
        m->pf_one_plane = m->dtype == SH_DTYPE_F16;
        const hipError_t e2 = enqueue_prefill(m, seq, seq, true, false);
        m->pf_one_plane = false;
        const hipError_t e3 = hipStreamEndCapture(m->stream, &g);
        if (!hip_ok(e2, "prefill") || !hip_ok(e3, "end capture")) {
            if (g) (void)hipGraphDestroy(g);
            return -1;
        }
        const hipError_t e4 = hipGraphInstantiate(&m->pf_exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (!hip_ok(e4, "instantiate prefill")) return -1;
        m->pf_ready = true;
        m->pf_graph_seq = seq;
    }
    if (!hip_ok(hipEventRecord(m->ev0, m->stream), "event")) return -1;
    if (!hip_ok(hipGraphLaunch(m->pf_exec, m->stream), "prefill")) return -1;
    if (!hip_ok(hipEventRecord(m->ev1, m->stream), "event")) return -1;
    const size_t n = (size_t)m->cfg.vocab * seq;
    if (!hip_ok(hipMemcpyAsync(logits_cf, m->pf_logits, sizeof(float) * n,
                               hipMemcpyDeviceToHost, m->stream), "prefill logits"))
        return -1;
    if (!hip_ok(hipStreamSynchronize(m->stream), "prefill sync")) return -1;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, m->ev0, m->ev1);
    m->last.gpu_ms = ms;
    m->last.forwards = 1;
    m->last.tokens_out = seq;
    m->last.bytes_per_forward_mean = prefill_bytes(m, seq);
    m->last.persistent = 0;
    m->last.grid = 0;
    m->last.prefill_ms = ms;
    return 0;
}

// Algorithmic bytes of one batched step with every sequence at position pos: the weights once,
// then per sequence its K/V rows 0..pos read, one K/V row written, the logits written and
// read back by the argmax, and its embedding row.
double batch_step_bytes(const sh_model *m, int B, int pos) {
    const sh_config &c = m->cfg;
    const double eb = (double)weight_elem_bytes(m->dtype);
    const double D = c.dim, F = c.hidden, Q = m->qdim, KV = m->kvdim;
    double w = (eb * ((Q + 2 * KV) * D + D * Q + 2 * F * D + D * F) + 4.0 * 2 * D) * c.n_layers;
    if (c.qk_norm) w += 4.0 * 2 * c.head_dim * c.n_layers;
    w += eb * (double)c.vocab * D + 4.0 * D;
    const double kvb = (double)kv_elem_bytes(c.kv_dtype);
    const double per_seq = kvb * 2 * KV * c.n_layers * (double)(pos + 2) + 8.0 * c.vocab + 2.0 * D;
    return w + B * per_seq;
}

// The batched decode; with keep_rows, the logits of sequences keep_rows[0, n_keep) are copied
// out after every step into keep_out[(step * n_keep + i) * vocab] (the steps then run as eager
// launches, not the captured step graph).
static int batch_greedy_decode(sh_model *m, const int32_t *prompts, int32_t n_seqs, int32_t prompt_len,
                               int32_t max_new, int32_t *out_tokens, int32_t *n_out, const int32_t *keep_rows,
                               int32_t n_keep, float *keep_out) {
    if (!ready(m)) return -1;
    const sh_config &c = m->cfg;
    if (!prompts || !out_tokens || !n_out || n_seqs < 1 || prompt_len < 1 ||
        prompt_len > c.max_seq) {
        set_error("sh_batch_greedy_decode: bad arguments");
        return -1;
    }
    std::string why;
    if (!batch_supported(m, n_seqs, &why)) {
        set_error("sh_batch_greedy_decode: " + why);
        return -1;
    }
    for (size_t i = 0; i < (size_t)n_seqs * prompt_len; i++)
        if (prompts[i] < 0 || prompts[i] >= c.vocab) {   // infer.go:160-163
            set_error("sh_batch_greedy_decode: prompt token[" + std::to_string(i % prompt_len) +
                      "] of sequence " + std::to_string(i / prompt_len) + " out of range");
            return -1;
        }
    if (max_new <= 0) max_new = 64;                       // infer.go:140-143
    const int B = n_seqs, P = prompt_len;
    const int steps = std::min(max_new, c.max_seq - P);   // stop at len == maxSeq
    for (int i = 0; i < n_keep; i++)
        if (keep_rows[i] < 0 || keep_rows[i] >= B) {
            set_error("sh_batch_greedy_decode_logits: sequence " + std::to_string(keep_rows[i]) + " out of range");
            return -1;
        }
    (void)hipSetDevice(m->device);
    if (!hip_ok(batch_alloc(m, B), "batch scratch") || !hip_ok(batch_new_generation(m), "batch generation"))
        return -1;
    float *keep_dev = nullptr;
    const size_t keep_floats = (size_t)std::max(steps, 1) * n_keep * c.vocab;
    if (n_keep > 0 && !hip_ok(hipMalloc(&keep_dev, 4 * keep_floats), "logits buffer")) return -1;
    struct Free {
        float *p;
        ~Free() { (void)hipFree(p); }
    } free_keep{keep_dev};
    hipStream_t s = m->stream;
    // prompt rows 0..P-2 of every sequence: one causal forward that fills the caches
    const int S = B * (P - 1);
    std::vector<int32_t> rows(3 * (size_t)std::max(S, 1));
    if (S > 0) {
        if (!hip_ok(prefill_alloc(m, S, false), "prefill scratch")) return -1;
        for (int b = 0; b < B; b++)
            for (int t = 0; t < P - 1; t++) {
                const size_t r = (size_t)b * (P - 1) + t;
                rows[r] = prompts[(size_t)b * P + t];
                rows[S + r] = t;
                rows[2 * (size_t)S + r] = b;
            }
        if (!hip_ok(hipMemcpyAsync(m->pf_tokens, rows.data(), 4 * (size_t)S, hipMemcpyHostToDevice, s), "rows") ||
            !hip_ok(hipMemcpyAsync(m->pf_rowpos, rows.data() + S, 4 * (size_t)S, hipMemcpyHostToDevice, s), "rows") ||
            !hip_ok(hipMemcpyAsync(m->pf_rowseq, rows.data() + 2 * (size_t)S, 4 * (size_t)S, hipMemcpyHostToDevice, s), "rows"))
            return -1;
    }
    // device state: token P-1 at position P-1 next; history rows start with the prompt
    const size_t hs = (size_t)c.max_seq + 1;
    std::vector<int32_t> hist((size_t)B * hs, 0), tok(B), pos(B, P - 1);
    for (int b = 0; b < B; b++) {
        memcpy(&hist[(size_t)b * hs], prompts + (size_t)b * P, 4 * (size_t)P);
        tok[b] = prompts[(size_t)b * P + P - 1];
    }
    if (!hip_ok(hipMemcpyAsync(m->bt_hist, hist.data(), 4 * hist.size(), hipMemcpyHostToDevice, s), "hist") ||
        !hip_ok(hipMemcpyAsync(m->bt_tok, tok.data(), 4 * (size_t)B, hipMemcpyHostToDevice, s), "tok") ||
        !hip_ok(hipMemcpyAsync(m->bt_pos, pos.data(), 4 * (size_t)B, hipMemcpyHostToDevice, s), "pos"))
        return -1;
    if (!m->bt_ready || m->bt_graph_b != B) {
        if (m->bt_ready) (void)hipGraphExecDestroy(m->bt_exec);
        m->bt_ready = false;
        hipGraph_t g = nullptr;
        if (!hip_ok(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "capture")) return -1;
        const hipError_t e2 = enqueue_batch_step(m, B);
        const hipError_t e3 = hipStreamEndCapture(s, &g);
        if (!hip_ok(e2, "batch step") || !hip_ok(e3, "end capture")) {
            if (g) (void)hipGraphDestroy(g);
            return -1;
        }
        const hipError_t e4 = hipGraphInstantiate(&m->bt_exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (!hip_ok(e4, "instantiate batch step")) return -1;
        m->bt_ready = true;
        m->bt_graph_b = B;
    }
    hipEvent_t e0 = m->ev0, e1 = m->ev1, e2 = nullptr;
    if (!hip_ok(hipEventCreate(&e2), "event")) return -1;
    bool ok = hip_ok(hipMemsetAsync(m->bt_err, 0, 4, s), "clear error word") && hip_ok(hipEventRecord(e0, s), "event");
    if (ok && S > 0) ok = hip_ok(enqueue_prefill(m, S, P - 1, false, true), "batch prefill");
    ok = ok && hip_ok(hipEventRecord(e1, s), "event");
    for (int i = 0; ok && i < steps; i++) {
        if (n_keep == 0) {
            ok = hip_ok(hipGraphLaunch(m->bt_exec, s), "batch step");
            continue;
        }
        ok = hip_ok(enqueue_batch_step(m, B), "batch step");
        for (int k = 0; ok && k < n_keep; k++)
            ok = hip_ok(hipMemcpyAsync(keep_dev + ((size_t)i * n_keep + k) * c.vocab,
                                       m->bt_logits + (size_t)keep_rows[k] * c.vocab, 4 * (size_t)c.vocab,
                                       hipMemcpyDeviceToDevice, s),
                        "keep logits");
    }
    ok = ok && hip_ok(hipEventRecord(e2, s), "event") && hip_ok(hipStreamSynchronize(s), "batch sync");
    if (ok && n_keep > 0)
        ok = hip_ok(hipMemcpy(keep_out, keep_dev, 4 * (size_t)steps * n_keep * c.vocab, hipMemcpyDeviceToHost),
                    "read logits");
    ok = ok && hip_ok(hipMemcpy(hist.data(), m->bt_hist, 4 * hist.size(), hipMemcpyDeviceToHost), "read tokens");
    int32_t lost = 0;
    ok = ok && hip_ok(hipMemcpy(&lost, m->bt_err, 4, hipMemcpyDeviceToHost), "read error word");
    if (ok && lost) {
        set_error("sh_batch_greedy_decode: an attention split's partial never arrived (bounded wait expired)");
        ok = false;
    }
    float pre_ms = 0, dec_ms = 0;
    if (ok) {
        (void)hipEventElapsedTime(&pre_ms, e0, e1);
        (void)hipEventElapsedTime(&dec_ms, e1, e2);
    }
    (void)hipEventDestroy(e2);
    if (!ok) return -1;
    const size_t stride = (size_t)P + max_new;
    int64_t kept = 0;
    for (int b = 0; b < B; b++) {
        int n = P + steps;
        for (int i = P; i < P + steps; i++)
            if (hist[(size_t)b * hs + i] == kEos) {   // infer.go:189-192: EOS is kept
                n = i + 1;
                break;
            }
        memcpy(out_tokens + (size_t)b * stride, &hist[(size_t)b * hs], 4 * (size_t)n);
        n_out[b] = n;
        kept += n - P;
    }
    double bytes = 0;
    for (int i = 0; i < steps; i++) bytes += batch_step_bytes(m, B, P - 1 + i);
    m->last.gpu_ms = dec_ms;
    m->last.prefill_ms = pre_ms;
    m->last.forwards = steps;
    m->last.tokens_out = kept;
    m->last.bytes_per_forward_mean = steps ? bytes / steps : 0;
    m->last.persistent = 0;
    m->last.grid = 0;
    return 0;
}

int sh_batch_greedy_decode(sh_model *m, const int32_t *prompts, int32_t n_seqs, int32_t prompt_len,
                           int32_t max_new, int32_t *out_tokens, int32_t *n_out) {
    return batch_greedy_decode(m, prompts, n_seqs, prompt_len, max_new, out_tokens, n_out, nullptr, 0, nullptr);
}

int sh_batch_greedy_decode_logits(sh_model *m, const int32_t *prompts, int32_t n_seqs, int32_t prompt_len,
                                  int32_t max_new, int32_t *out_tokens, int32_t *n_out, const int32_t *rows,
                                  int32_t n_rows, float *logits_out) {
    if (!rows || n_rows < 1 || !logits_out) {
        set_error("sh_batch_greedy_decode_logits: bad arguments");
        return -1;
    }
    return batch_greedy_decode(m, prompts, n_seqs, prompt_len, max_new, out_tokens, n_out, rows, n_rows,
                               logits_out);
}

int sh_window_greedy_decode(sh_model *m, const int32_t *prompt, int32_t n_prompt, int32_t seq,
                            int32_t max_new, int32_t *out_tokens, int32_t *n_out,
                            int32_t *stopped_eos) {
    if (!ready(m)) return -1;
    const sh_config &c = m->cfg;
    if ((!prompt && n_prompt > 0) || n_prompt < 0 || !out_tokens || !n_out || !stopped_eos ||
        seq < 1 || seq > c.max_seq) {
        set_error("sh_window_greedy_decode: bad arguments");
        return -1;
    }
    std::string why;
    if (!prefill_supported(m, &why)) {
        set_error("sh_window_greedy_decode: " + why);
        return -1;
    }
    if (max_new <= 0) max_new = 64;                         // decode.go:22-25
    std::vector<int32_t> toks;                              // decode.go:35-46
    if (n_prompt == 0) toks.push_back(kBos);
    else toks.assign(prompt + (n_prompt > seq ? n_prompt - seq : 0), prompt + n_prompt);
    for (size_t i = 0; i < toks.size(); i++)
        if (toks[i] < 0 || toks[i] >= c.vocab) {
            set_error("sh_window_greedy_decode: prompt token[" + std::to_string(i) + "]=" +
                      std::to_string(toks[i]) + " out of range");
            return -1;
        }
    const int P = (int)toks.size();
    (void)hipSetDevice(m->device);
    if (!hip_ok(prefill_alloc(m, seq, false), "window scratch") ||
        !hip_ok(window_alloc(m, max_new), "window scratch"))
        return -1;
    hipStream_t s = m->stream;
    // the window (fillDecodeWindow), rows at positions 0..seq-1 of one sequence
    std::vector<int32_t> rows(3 * (size_t)seq, kBos);
    for (int i = 0; i < P; i++) rows[seq - P + i] = toks[i];
    for (int t = 0; t < seq; t++) {
        rows[seq + t] = t;
        rows[2 * (size_t)seq + t] = 0;
    }
    const int32_t zero = 0;
    if (!hip_ok(hipMemcpyAsync(m->pf_tokens, rows.data(), 4 * (size_t)seq, hipMemcpyHostToDevice, s), "window") ||
        !hip_ok(hipMemcpyAsync(m->pf_rowpos, rows.data() + seq, 4 * (size_t)seq, hipMemcpyHostToDevice, s), "window") ||
        !hip_ok(hipMemcpyAsync(m->pf_rowseq, rows.data() + 2 * (size_t)seq, 4 * (size_t)seq, hipMemcpyHostToDevice, s), "window") ||
        !hip_ok(hipMemcpyAsync(m->wd_count, &zero, 4, hipMemcpyHostToDevice, s), "window"))
        return -1;
    if (!m->wd_ready || m->wd_seq != seq) {
        if (m->wd_ready) (void)hipGraphExecDestroy(m->wd_exec);
        m->wd_ready = false;
        hipGraph_t g = nullptr;
        if (!hip_ok(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "capture")) return -1;
        const hipError_t e2 = enqueue_window_step(m, seq);
        const hipError_t e3 = hipStreamEndCapture(s, &g);
        if (!hip_ok(e2, "window step") || !hip_ok(e3, "end capture")) {
            if (g) (void)hipGraphDestroy(g);
            return -1;
        }
        const hipError_t e4 = hipGraphInstantiate(&m->wd_exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (!hip_ok(e4, "instantiate window step")) return -1;
        m->wd_ready = true;
        m->wd_seq = seq;
    }
    bool ok = hip_ok(hipEventRecord(m->ev0, s), "event");
    for (int i = 0; ok && i < max_new; i++) ok = hip_ok(hipGraphLaunch(m->wd_exec, s), "window step");
    ok = ok && hip_ok(hipEventRecord(m->ev1, s), "event") && hip_ok(hipStreamSynchronize(s), "window sync");
    std::vector<int32_t> gen(max_new);
    ok = ok && hip_ok(hipMemcpy(gen.data(), m->wd_hist, 4 * (size_t)max_new, hipMemcpyDeviceToHost), "read tokens");
    if (!ok) return -1;
    memcpy(out_tokens, toks.data(), 4 * (size_t)P);
    int n = P, eos = 0;
    for (int i = 0; i < max_new; i++) {
        out_tokens[n++] = gen[i];
        if (gen[i] == kEos) {   // decode.go:66-69: EOS is kept, the loop ends
            eos = 1;
            break;
        }
    }
    *n_out = n;
    *stopped_eos = eos;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, m->ev0, m->ev1);
    m->last.gpu_ms = ms;
    m->last.forwards = max_new;
    m->last.tokens_out = n - P;
    m->last.bytes_per_forward_mean = prefill_bytes(m, seq);
    m->last.persistent = 0;
    m->last.grid = 0;
    m->last.prefill_ms = 0;
    return 0;
}

int sh_decode_tap(const sh_model *m, int32_t which, float *out, int32_t n) {
    if (!m || !out) {
        set_error("sh_decode_tap: bad arguments");
        return -1;
    }
    const sh_config &c = m->cfg;
    int len = 0;
    const float *dense = nullptr;      // per-stage path buffers (fp32)
    const uint64_t *words = nullptr;   // persistent path hand-over words (value | epoch)
    switch (which) {
    case SH_TAP_X: len = c.dim; dense = m->x; words = m->ll_x; break;
    case SH_TAP_QKV: len = m->qkv_rows; dense = m->qkv; words = m->ll_qkv; break;
    case SH_TAP_ATT: len = m->qdim; dense = m->att; words = m->ll_att; break;
    case SH_TAP_GATE: len = c.hidden; dense = m->gate; words = m->ll_gate; break;
    case SH_TAP_X2: len = c.dim; dense = m->x2; words = m->ll_x2; break;
    default:
        set_error("sh_decode_tap: unknown tap");
        return -1;
    }
    if (n != len) {
        set_error("sh_decode_tap: n must be " + std::to_string(len));
        return -1;
    }
    (void)hipSetDevice(m->device);
    if (!hip_ok(hipStreamSynchronize(m->stream), "tap sync")) return -1;
    if (m->persistent) {
        // x, x2 and the gate vector are stored in padded blocks, one per producer workgroup
        int st = -1;
        if (which == SH_TAP_X) st = 3;
        if (which == SH_TAP_X2) st = 1;
        if (which == SH_TAP_GATE) st = 2;
        const int per = st < 0 ? len : (st == 2 ? m->p_own[2].per / 2 : m->p_own[st].per);
        const int stride = st < 0 ? len : m->p_ostride[st];
        const size_t nw = st < 0 ? (size_t)len : stage_words(m, st);
        std::vector<uint64_t> w(nw);
        if (!hip_ok(hipMemcpy(w.data(), words, 8 * nw, hipMemcpyDeviceToHost), "tap read"))
            return -1;
        for (int i = 0; i < len; i++) {
            const uint32_t b = (uint32_t)w[(size_t)(i / per) * stride + i % per];
            memcpy(&out[i], &b, 4);
        }
        return 0;
    }
    return hip_ok(hipMemcpy(out, dense, 4 * (size_t)len, hipMemcpyDeviceToHost), "tap read") ? 0 : -1;
}

int sh_debug_option(sh_model *m, int32_t option, int32_t value) {
    if (!m) {
        set_error("sh_debug_option: nil model");
        return -1;
    }
    if (option == SH_DEBUG_FAIL_NEXT_LAUNCH) {
        if (!m->persistent) {
            set_error("sh_debug_option: the model does not run the persistent decode kernel");
            return -1;
        }
        if (value != 0 && value != kErrTimeout && value != kErrAbsent) {
            set_error("sh_debug_option: SH_DEBUG_FAIL_NEXT_LAUNCH takes 0 (off), 1 (a wait timed out with "
                      "every workgroup running) or 2 (the grid was not all resident)");
            return -1;
        }
        m->fail_next = value;
        return 0;
    }
    if (option == SH_DEBUG_PROMPT_PREFILL) {
        m->no_prompt_prefill = value == 0;
        return 0;
    }
    set_error("sh_debug_option: unknown option " + std::to_string(option));
    return -1;
}

int sh_trace_forward(sh_model *m, int32_t forward) {
    if (!m || !m->persistent) {
        set_error("sh_trace_forward: tracing needs the persistent decode kernel");
        return -1;
    }
    m->trace_f = forward < 0 ? -1 : forward;
    return 0;
}

int sh_trace_read(sh_model *m, int64_t *out, int32_t cap, int32_t *n_out, double *ticks_per_s) {
    if (!m || !m->persistent || !out || !n_out || !ticks_per_s) {
        set_error("sh_trace_read: bad arguments");
        return -1;
    }
    const int n = m->p_grid * 2 * (5 * m->cfg.n_layers + 3);
    if (cap < n) {
        set_error("sh_trace_read: capacity below grid*2*(5*n_layers+3)");
        return -1;
    }
    (void)hipSetDevice(m->device);
    if (!hip_ok(hipMemcpy(out, m->trace_buf, sizeof(int64_t) * n, hipMemcpyDeviceToHost), "read trace"))
        return -1;
    int rate_khz = 0;
    if (!hip_ok(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, m->device), "clock rate"))
        return -1;
    *n_out = n;
    *ticks_per_s = (double)rate_khz * 1000.0;
    return 0;
}

size_t sh_model_describe(const sh_model *m, char *buf, size_t len) {
    const std::string d = m ? std::string(m->path_note) : std::string("nil model");
    if (buf && len) {
        const size_t n = std::min(len - 1, d.size());
        memcpy(buf, d.data(), n);
        buf[n] = 0;
    }
    return d.size();
}

int sh_stats(const sh_model *m, sh_timing *out) {
    if (!m || !out) {
        set_error("sh_stats: nil argument");
        return -1;
    }
    *out = m->last;
    return 0;
}

int sh_quantize_i8(const float *src, int32_t rows, int32_t cols, int8_t *dst, float *scales,
                   int32_t per_row) {
    if (rows < 0 || cols < 0 || (!src && rows * cols) || (!dst && rows * cols) || !scales) {
        set_error("sh_quantize_i8: bad arguments");
        return -1;
    }
    (void)hipSetDevice(g_device);
    const size_t n = (size_t)rows * cols;
    const size_t ns = per_row ? (size_t)std::max(rows, 1) : 1;
    float *dsrc = nullptr, *dsc = nullptr, *work = nullptr;
    int8_t *ddst = nullptr;
    int rc = -1;
    if (hip_ok(hipMalloc(&dsrc, std::max<size_t>(n, 1) * 4), "hipMalloc") &&
        hip_ok(hipMalloc(&ddst, std::max<size_t>(n, 1)), "hipMalloc") &&
        hip_ok(hipMalloc(&dsc, ns * 4), "hipMalloc") && hip_ok(hipMalloc(&work, 16), "hipMalloc") &&
        (n == 0 || hip_ok(hipMemcpy(dsrc, src, n * 4, hipMemcpyHostToDevice), "copy src"))) {
        hipError_t e = per_row ? launch_quantize_rows(dsrc, ddst, dsc, rows, cols, 1, 0, 1, 0, nullptr)
                               : launch_quantize_tensor(dsrc, ddst, dsc, n, work, nullptr);
        if (hip_ok(e, "quantize") && hip_ok(hipDeviceSynchronize(), "quantize sync") &&
            (n == 0 || hip_ok(hipMemcpy(dst, ddst, n, hipMemcpyDeviceToHost), "copy q")) &&
            hip_ok(hipMemcpy(scales, dsc, (per_row ? (size_t)rows : 1) * 4, hipMemcpyDeviceToHost),
                   "copy scales"))
            rc = 0;
    }
    (void)hipFree(dsrc);
    (void)hipFree(ddst);
    (void)hipFree(dsc);
    (void)hipFree(work);
    return rc;
}

int sh_dequantize_i8(const int8_t *q, const float *scales, int32_t rows, int32_t cols,
                     int32_t per_row, float *dst) {
    if (rows < 0 || cols < 0 || !scales || ((!q || !dst) && rows * cols)) {
        set_error("sh_dequantize_i8: bad arguments");
        return -1;
    }
    const size_t n = (size_t)rows * cols;
    if (n == 0) return 0;
    (void)hipSetDevice(g_device);
    const size_t ns = per_row ? (size_t)rows : 1;
    int8_t *dq = nullptr;
    float *ds = nullptr, *dd = nullptr;
    int rc = -1;
    if (hip_ok(hipMalloc(&dq, n), "hipMalloc") && hip_ok(hipMalloc(&ds, ns * 4), "hipMalloc") &&
        hip_ok(hipMalloc(&dd, n * 4), "hipMalloc") &&
        hip_ok(hipMemcpy(dq, q, n, hipMemcpyHostToDevice), "copy q") &&
        hip_ok(hipMemcpy(ds, scales, ns * 4, hipMemcpyHostToDevice), "copy scales") &&
        hip_ok(launch_dequantize(dq, ds, rows, cols, per_row, dd, nullptr), "dequantize") &&
        hip_ok(hipDeviceSynchronize(), "dequantize sync") &&
        hip_ok(hipMemcpy(dst, dd, n * 4, hipMemcpyDeviceToHost), "copy dst"))
        rc = 0;
    (void)hipFree(dq);
    (void)hipFree(ds);
    (void)hipFree(dd);
    return rc;
}

int sh_synth_normal(float *dst, size_t n, uint64_t seed, uint64_t tensor_id, float std_) {
    if (!dst && n) {
        set_error("sh_synth_normal: nil destination");
        return -1;
    }
    const uint64_t key = splitmix64(seed ^ splitmix64(tensor_id + 0x632BE59BD9B4E019ull));
    parallel_ranges(n, [=](size_t a, size_t b) {
        const double two_pi = 6.283185307179586476925286766559;
        for (size_t i = a; i < b; i++) {
            const uint64_t r1 = splitmix64(key + 2 * (uint64_t)i);
            const uint64_t r2 = splitmix64(key + 2 * (uint64_t)i + 1);
            const double u1 = (double)((r1 >> 11) + 1) * (1.0 / 9007199254740992.0);
            const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
            const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
            dst[i] = (float)(z * (double)std_);
        }
    });
    return 0;
}

int sh_copy_calibrate(size_t bytes, int32_t reps, double *ms_per_copy, double *gbps) {
    if (bytes == 0 || bytes % 16 || reps <= 0 || !ms_per_copy || !gbps) {
        set_error("sh_copy_calibrate: bytes must be a positive multiple of 16, reps > 0");
        return -1;
    }
    void *a = nullptr, *b = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool ok = hip_ok(hipMalloc(&a, bytes), "calibrate alloc") &&
              hip_ok(hipMalloc(&b, bytes), "calibrate alloc") &&
              hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "calibrate stream") &&
              hip_ok(hipEventCreate(&e0), "calibrate event") &&
              hip_ok(hipEventCreate(&e1), "calibrate event") &&
              hip_ok(hipMemsetAsync(a, 0x5a, bytes, s), "calibrate fill") &&
              hip_ok(launch_copy_calibrate(a, b, bytes, s), "calibrate copy") &&
              hip_ok(hipEventRecord(e0, s), "calibrate event");
    for (int r = 0; ok && r < reps; r++) ok = hip_ok(launch_copy_calibrate(a, b, bytes, s), "calibrate copy");
    ok = ok && hip_ok(hipEventRecord(e1, s), "calibrate event") &&
         hip_ok(hipStreamSynchronize(s), "calibrate sync");
    float ms = 0;
    if (ok) ok = hip_ok(hipEventElapsedTime(&ms, e0, e1), "calibrate time");
    if (ok) {
        *ms_per_copy = ms / reps;
        *gbps = 2.0 * (double)bytes / (*ms_per_copy * 1e-3) / 1e9;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    (void)hipFree(a);
    (void)hipFree(b);
    return ok ? 0 : -1;
}

int sh_read_calibrate(size_t bytes, int32_t reps, double *ms_per_read, double *gbps) {
    if (bytes == 0 || bytes % 16 || reps <= 0 || !ms_per_read || !gbps) {
        set_error("sh_read_calibrate: bytes must be a positive multiple of 16, reps > 0");
        return -1;
    }
    void *a = nullptr;
    uint32_t *out = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    // every 16-byte word holds 0x5a5a5a5a four times, so the XOR the kernel folds is 0 or
    // 0x5a5a5a5a, never 0xffffffff
    const uint32_t never = 0xffffffffu;
    bool ok = hip_ok(hipMalloc(&a, bytes), "calibrate alloc") &&
              hip_ok(hipMalloc(&out, sizeof(uint32_t)), "calibrate alloc") &&
              hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "calibrate stream") &&
              hip_ok(hipEventCreate(&e0), "calibrate event") &&
              hip_ok(hipEventCreate(&e1), "calibrate event") &&
              hip_ok(hipMemsetAsync(a, 0x5a, bytes, s), "calibrate fill") &&
              hip_ok(launch_read_calibrate(a, bytes, never, out, s), "calibrate read") &&
              hip_ok(hipEventRecord(e0, s), "calibrate event");
    for (int r = 0; ok && r < reps; r++) ok = hip_ok(launch_read_calibrate(a, bytes, never, out, s), "calibrate read");
    ok = ok && hip_ok(hipEventRecord(e1, s), "calibrate event") &&
         hip_ok(hipStreamSynchronize(s), "calibrate sync");
    float ms = 0;
    if (ok) ok = hip_ok(hipEventElapsedTime(&ms, e0, e1), "calibrate time");
    if (ok) {
        *ms_per_read = ms / reps;
        *gbps = (double)bytes / (*ms_per_read * 1e-3) / 1e9;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    (void)hipFree(a);
    (void)hipFree(out);
    return ok ? 0 : -1;
}

int sh_synth_tokens(int32_t *dst, size_t n, uint64_t seed, int32_t vocab) {
    if ((!dst && n) || vocab <= 0) {
        set_error("sh_synth_tokens: bad arguments");
        return -1;
    }
    const uint64_t key = splitmix64(seed ^ 0x7A3C15E2D4B9F681ull);
    for (size_t i = 0; i < n; i++) dst[i] = (int32_t)(splitmix64(key + i) % (uint64_t)vocab);
    return 0;
}

int sh_round_dtype(float *data, size_t n, int32_t dtype) {
    if (!data && n) {
        set_error("sh_round_dtype: nil data");
        return -1;
    }
    if (dtype != SH_DTYPE_F16 && dtype != SH_DTYPE_BF16) {
        set_error("sh_round_dtype: dtype must be SH_DTYPE_F16 or SH_DTYPE_BF16");
        return -1;
    }
    parallel_ranges(n, [=](size_t a, size_t b) {
        for (size_t i = a; i < b; i++) {
            if (dtype == SH_DTYPE_BF16) {
                const uint32_t u = (uint32_t)host_bf16_bits(data[i]) << 16;
                memcpy(&data[i], &u, 4);
            } else {
                data[i] = (float)(_Float16)data[i];
            }
        }
    });
    return 0;
}

int sh_layer_forward_cf(sh_model *m, int32_t layer, const float *x_cf, int32_t seq,
                        float *out_cf) {
    if (m && (layer < 0 || layer >= m->cfg.n_layers)) {
        set_error("sh_layer_forward_cf: layer out of range");
        return -1;
    }
    if (!seam_begin(m, "sh_layer_forward_cf", x_cf, seq, out_cf, false, false)) return -1;
    if (!hip_ok(enqueue_layer_cf(m, layer, seq), "layer forward")) return -1;
    return seam_end(m, m->pf_cf, out_cf, sizeof(float) * (size_t)m->cfg.dim * seq, seq) ? 0 : -1;
}

int sh_layer_forward_cf_taps(sh_model *m, int32_t layer, const float *x_cf, int32_t seq,
                             float *out_cf, float *sdpa_cf, float *ffn_cf) {
    if (m && (layer < 0 || layer >= m->cfg.n_layers)) {
        set_error("sh_layer_forward_cf_taps: layer out of range");
        return -1;
    }
    if (!seam_begin(m, "sh_layer_forward_cf_taps", x_cf, seq, out_cf, false, false)) return -1;
    const sh_config &c = m->cfg;
    const size_t S = (size_t)seq;
    const size_t n_sdpa = (size_t)(c.dim + 2 * m->qdim + 2 * m->kvdim) * S;
    const size_t n_ffn = (size_t)(c.dim + 2 * c.hidden) * S;
    const size_t n_h13 = 2 * (size_t)c.hidden * S;
    const size_t need = n_sdpa + n_ffn + n_h13;
    if (m->tap_cap < need) {
        (void)hipFree(m->tap_buf);
        m->tap_buf = nullptr;
        m->tap_cap = 0;
        if (!hip_ok(hipMalloc(&m->tap_buf, sizeof(float) * need), "tap scratch")) return -1;
        m->tap_cap = need;
    }
    float *d_sdpa = m->tap_buf, *d_ffn = d_sdpa + n_sdpa, *d_h13 = d_ffn + n_ffn;
    if (!hip_ok(enqueue_layer_cf(m, layer, seq), "layer forward") ||
        !hip_ok(enqueue_layer_taps_cf(m, layer, seq, sdpa_cf ? d_sdpa : nullptr, ffn_cf ? d_ffn : nullptr,
                                      d_h13), "layer taps"))
        return -1;
    if (sdpa_cf && !hip_ok(hipMemcpyAsync(sdpa_cf, d_sdpa, sizeof(float) * n_sdpa, hipMemcpyDeviceToHost,
                                          m->stream), "sdpa taps"))
        return -1;
    if (ffn_cf && !hip_ok(hipMemcpyAsync(ffn_cf, d_ffn, sizeof(float) * n_ffn, hipMemcpyDeviceToHost,
                                         m->stream), "ffn taps"))
        return -1;
    return seam_end(m, m->pf_cf, out_cf, sizeof(float) * (size_t)c.dim * seq, seq) ? 0 : -1;
}

int sh_rms_final_cf(sh_model *m, const float *x_cf, int32_t seq, float *out_cf) {
    if (!seam_begin(m, "sh_rms_final_cf", x_cf, seq, out_cf, false, true)) return -1;
    if (!hip_ok(enqueue_rms_final_cf(m, seq), "final rmsnorm")) return -1;
    return seam_end(m, m->pf_cf, out_cf, sizeof(float) * (size_t)m->cfg.dim * seq, seq) ? 0 : -1;
}

int sh_classifier_cf(sh_model *m, const float *xnorm_cf, int32_t seq, float *logits_cf) {
    if (!seam_begin(m, "sh_classifier_cf", xnorm_cf, seq, logits_cf, true, true)) return -1;
    if (!hip_ok(enqueue_classifier_cf(m, seq), "classifier")) return -1;
    return seam_end(m, m->pf_logits, logits_cf, sizeof(float) * (size_t)m->cfg.vocab * seq, seq) ? 0 : -1;
}

int sh_matmul_vocab_seq(const float *embed, const float *x_cf, int32_t vocab, int32_t dim,
                        int32_t seq, float *logits_cf) {
    if (!embed || !x_cf || !logits_cf || vocab <= 0 || dim <= 0 || seq <= 0) {
        set_error("sh_matmul_vocab_seq: bad arguments");
        return -1;
    }
    if (dim % 32 || vocab % 64) {
        set_error("sh_matmul_vocab_seq: needs dim % 32 == 0 and vocab % 64 == 0");
        return -1;
    }
    (void)hipSetDevice(g_device);
    const size_t V = vocab, D = dim, S = seq;
    const size_t part = gemm_partial_elems(seq, vocab, dim);
    float *e32 = nullptr, *xcf = nullptr, *xr = nullptr, *lg = nullptr, *pp = nullptr;
    uint16_t *w16 = nullptr, *planes = nullptr;
    int rc = -1;
    if (hip_ok(hipMalloc(&e32, 4 * V * D), "hipMalloc") && hip_ok(hipMalloc(&w16, 2 * V * D), "hipMalloc") &&
        hip_ok(hipMalloc(&xcf, 4 * D * S), "hipMalloc") && hip_ok(hipMalloc(&xr, 4 * D * S), "hipMalloc") &&
        hip_ok(hipMalloc(&planes, 4 * D * S), "hipMalloc") && hip_ok(hipMalloc(&lg, 4 * V * S), "hipMalloc") &&
        (part == 0 || hip_ok(hipMalloc(&pp, 4 * part), "hipMalloc")) &&
        hip_ok(hipMemcpy(e32, embed, 4 * V * D, hipMemcpyHostToDevice), "copy embed") &&
        hip_ok(hipMemcpy(xcf, x_cf, 4 * D * S, hipMemcpyHostToDevice), "copy x") &&
        hip_ok(launch_convert_rows(e32, w16, vocab, dim, SH_DTYPE_F16, 1, 0, nullptr), "convert embed") &&
        hip_ok(enqueue_transpose(xcf, dim, seq, xr, nullptr), "transpose x") &&
        hip_ok(enqueue_linear_rows(xr, seq, dim, w16, vocab, SH_DTYPE_F16, planes, lg, true, pp, part, nullptr),
               "vocab matmul") &&
        hip_ok(hipDeviceSynchronize(), "vocab matmul sync") &&
        hip_ok(hipMemcpy(logits_cf, lg, 4 * V * S, hipMemcpyDeviceToHost), "copy logits"))
        rc = 0;
    (void)hipFree(e32);
    (void)hipFree(w16);
    (void)hipFree(xcf);
    (void)hipFree(xr);
    (void)hipFree(planes);
    (void)hipFree(lg);
    (void)hipFree(pp);
    return rc;
}

}  // extern "C"

struct sh_conv {
    int out_dim, in_dim, device;
    uint16_t *w;   // [out_dim, in_dim] fp16 bits
};

extern "C" {

sh_conv *sh_conv_create(const float *w, int32_t out_dim, int32_t in_dim) {
    if (!w || out_dim <= 0 || in_dim <= 0) {
        set_error("sh_conv_create: bad arguments");
        return nullptr;
    }
    if (in_dim % 32 || out_dim % 64) {
        set_error("sh_conv_create: needs in_dim % 32 == 0 and out_dim % 64 == 0");
        return nullptr;
    }
    (void)hipSetDevice(g_device);
    if (!hip_ok(gemm_setup(), "GEMM set-up")) return nullptr;
    const size_t n = (size_t)out_dim * in_dim;
    float *w32 = nullptr;
    sh_conv *c = new sh_conv{out_dim, in_dim, g_device, nullptr};
    const bool ok = hip_ok(hipMalloc(&c->w, 2 * n), "hipMalloc") && hip_ok(hipMalloc(&w32, 4 * n), "hipMalloc") &&
                    hip_ok(hipMemcpy(w32, w, 4 * n, hipMemcpyHostToDevice), "copy weights") &&
                    hip_ok(launch_convert_rows(w32, c->w, out_dim, in_dim, SH_DTYPE_F16, 1, 0, nullptr),
                           "convert weights") &&
                    hip_ok(hipDeviceSynchronize(), "conv create sync");
    (void)hipFree(w32);
    if (!ok) {
        sh_conv_destroy(c);
        return nullptr;
    }
    return c;
}

int sh_conv_eval(sh_conv *c, const float *x, int32_t s, float *out) {
    if (!c || !x || !out || s <= 0) {
        set_error("sh_conv_eval: bad arguments");
        return -1;
    }
    (void)hipSetDevice(c->device);
    const size_t S = s, I = c->in_dim, O = c->out_dim;
    const size_t part = gemm_partial_elems(s, c->out_dim, c->in_dim);
    float *xr = nullptr, *y = nullptr, *pp = nullptr;
    uint16_t *planes = nullptr;
    int rc = -1;
    if (hip_ok(hipMalloc(&xr, 4 * S * I), "hipMalloc") && hip_ok(hipMalloc(&planes, 4 * S * I), "hipMalloc") &&
        hip_ok(hipMalloc(&y, 4 * S * O), "hipMalloc") && (part == 0 || hip_ok(hipMalloc(&pp, 4 * part), "hipMalloc")) &&
        hip_ok(hipMemcpy(xr, x, 4 * S * I, hipMemcpyHostToDevice), "copy x") &&
        hip_ok(enqueue_linear_rows(xr, s, c->in_dim, c->w, c->out_dim, SH_DTYPE_F16, planes, y, false, pp, part,
                                   nullptr),
               "conv eval") &&
        hip_ok(hipDeviceSynchronize(), "conv eval sync") &&
        hip_ok(hipMemcpy(out, y, 4 * S * O, hipMemcpyDeviceToHost), "copy out"))
        rc = 0;
    (void)hipFree(xr);
    (void)hipFree(planes);
    (void)hipFree(y);
    (void)hipFree(pp);
    return rc;
}

int sh_conv_eval_noalloc(sh_conv *c, const float *x, int32_t s, float *out, void *stream) {
    if (!c || !x || !out || s <= 0) {
        set_error("sh_conv_eval_noalloc: bad arguments");
        return -1;
    }
    (void)hipSetDevice(c->device);
    const size_t plane_bytes = 2 * sizeof(uint16_t) * (size_t)s * c->in_dim;   // hi and lo planes
    const size_t part = gemm_partial_elems(s, c->out_dim, c->in_dim);
    const size_t part_off = align_up(plane_bytes, 256);
    const size_t need = part_off + sizeof(float) * part;
    if (need > kNoAllocScratchBytes) {
        set_error("sh_conv_eval_noalloc: s=" + std::to_string(s) + " needs " + std::to_string(need) +
                  " bytes of scratch; the allocation-free path holds " + std::to_string(kNoAllocScratchBytes));
        return -1;
    }
    uint8_t *base = (uint8_t *)scratch_address(c->device);
    if (!base) return -1;
    return hip_ok(enqueue_linear_rows(x, s, c->in_dim, c->w, c->out_dim, SH_DTYPE_F16, (uint16_t *)base, out, false,
                                      part ? (float *)(base + part_off) : nullptr, part, (hipStream_t)stream),
                  "conv eval (no alloc)")
               ? 0
               : -1;
}

void sh_conv_destroy(sh_conv *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipFree(c->w);
    delete c;
}

}  // extern "C"

namespace sh {
namespace {
uint16_t host_bf16_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
}  // namespace
}  // namespace sh
