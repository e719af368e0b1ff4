// model.cpp -- a resident whole-token decode step for a Qwen3-MoE GGUF: the
// weights uploaded once, activations and the KV cache never leaving the
// device, one synchronisation per token. The equivalent of the reference's
// DeviceModel::load / forward (crates/llamd-runtime/src/device.rs:262-722) and
// bit-identical to its CPU composition (crates/llamd-runtime/src/layer.rs:
// forward_layer + moe_ffn + forward):
//
//   x = embed(token)
//   per layer: attn_norm -> Q, K, V (Q6_K) -> per-head QK-norm -> RoPE ->
//              KV append -> attention -> O (Q6_K) -> ffn_inp = x + O ->
//              ffn_norm -> MoE (router, top-k, experts) -> x = ffn_inp + moe
//   logits = output (Q6_K) . (rms_norm(x) * output_norm); next = argmax
//
// Built only on the library's own C ABI and kernel launchers.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/llamd_hip.h"
#include "errors.hpp"
#include "launch.hpp"

using llamd::set_error;

namespace {

struct Layer {
    void *attn_q = nullptr, *attn_k = nullptr, *attn_v = nullptr, *attn_out = nullptr;  // Q6_K
    float *attn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *ffn_norm = nullptr;
    void *moe = nullptr;
    float *kc = nullptr, *vc = nullptr;  // [max_kv][kv_dim]
};

struct Model {
    int n_layer = 0, n_embd = 0, n_head = 0, n_head_kv = 0, hd = 0, n_vocab = 0, max_kv = 0;
    float eps = 0.0f, rope_base = 0.0f, scale = 0.0f;
    void *tok_embd = nullptr;      // ggml-layout Q6_K bytes, for the row lookup
    void *output = nullptr;        // Q6_K, tiled
    bool output_owned = false;
    float *output_norm = nullptr;
    void *lmhead = nullptr;
    std::vector<Layer> layers;
    float2 *rope = nullptr;        // [max_kv][hd/2] (cos, sin)
    // activations
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr,
          *o = nullptr, *ffn_inp = nullptr, *fn = nullptr, *logits = nullptr, *inv = nullptr;
    int8_t *aq = nullptr;
    float *ad = nullptr;
    int32_t *tokpos = nullptr, *next = nullptr;
    int32_t *stage = nullptr;       // page-locked host: token, position, next (async copies)
    hipGraphExec_t exec = nullptr;  // the captured step
    hipGraphExec_t exec_long = nullptr;  // the same with the split attention
    bool split_attn = false;        // attend_split for positions >= long_from
    int long_from = 0;
    float *scores = nullptr;        // [n_head][max_kv] (split attention)
    bool use_graph = true;
    bool fused_attn = false;        // attend_fused: QK-norm, RoPE, attention, Q8_K in one launch
    bool fused_norm = false;        // the FFN norm inside the MoE decode launch
    bool norm_qkv = false;          // the attention norm inside the Q/K/V launch
    bool prefetch = false;          // the O weights into L2 under the attention
    std::vector<void *> owned;     // device allocations to free
};

float *dalloc(Model &m, size_t bytes) {
    void *p = llamd_fwd_alloc(bytes);
    if (p) m.owned.push_back(p);
    return (float *)p;
}

bool get_u(void *g, const std::string &key, uint64_t *v) { return llamd_gguf_get_u64(g, key.c_str(), v) == 0; }

// an F32 tensor of exactly n values, copied to the device
float *upload_f32(Model &m, void *g, const std::string &name, uint64_t n) {
    const int64_t i = llamd_gguf_find_tensor(g, name.c_str());
    if (i < 0) { set_error("model: %s is absent", name.c_str()); return nullptr; }
    uint32_t type, nd;
    uint64_t dims[4], off, nb;
    if (llamd_gguf_tensor(g, (uint64_t)i, nullptr, 0, &nd, dims, &type, &off)) return nullptr;
    if (type != 0) { set_error("model: %s is type %u, expected F32", name.c_str(), type); return nullptr; }
    const void *src = llamd_gguf_tensor_data(g, (uint64_t)i, &nb);
    if (!src) return nullptr;
    if (nb != n * 4) { set_error("model: %s holds %llu values, expected %llu", name.c_str(), (unsigned long long)(nb / 4), (unsigned long long)n); return nullptr; }
    float *d = dalloc(m, nb);
    if (!d || llamd_fwd_upload(d, src, nb)) return nullptr;
    return d;
}

// Every launch of one token's step (embedding .. argmax) on stream st; the
// token and position come from m->tokpos.
bool enqueue_step(Model *m, hipStream_t st, bool long_ctx) {
    const int E = m->n_embd, eb = E / 256, qdim = m->n_head * m->hd, kv_dim = m->n_head_kv * m->hd;
    int rc = llamd::launch_embed_q6k(m->tok_embd, m->tokpos, eb, m->x, st);
    for (int il = 0; il < m->n_layer && !rc; ++il) {
        Layer &l = m->layers[il];
        // attn_norm = rms_norm(x) * w, quantized once for Q, K and V
        if (m->norm_qkv) {
            const void *wt[3] = {l.attn_q, l.attn_k, l.attn_v};
            float *const y[3] = {m->q, m->k, m->v};
            const int rows[3] = {qdim, kv_dim, kv_dim};
            rc |= llamd::launch_norm_qkv(m->x, l.attn_norm, m->eps, wt, y, rows, E, st);
        } else {
            llamd_fwd_rms_norm_quant(m->x, l.attn_norm, nullptr, m->aq, m->ad, m->inv, E, m->eps);
            llamd_fwd_matvec_x3(l.attn_q, l.attn_k, l.attn_v, m->aq, m->ad, m->q, m->k, m->v, eb,
                                qdim, kv_dim, kv_dim);
        }
        // QK-norm per head before RoPE (layer.rs:113-136), RoPE, KV append,
        // attention, and Q8_K of its output for the O projection
        if (long_ctx) {
            // long contexts: QK-norm, RoPE and the KV append, then the
            // logits over the whole GPU and the softmax / weighted V sum on
            // two workgroups per head, into the f32 attn (the same bits)
            rc |= llamd::launch_qk_norm_rope_store(m->q, m->k, m->v, l.q_norm, l.k_norm, m->rope,
                                                   m->tokpos + 1, m->n_head, m->n_head_kv, m->hd,
                                                   m->eps, l.kc, l.vc, st);
            rc |= llamd::launch_attend_split(m->q, l.kc, l.vc, m->tokpos + 1, m->n_head,
                                             m->n_head_kv, m->hd, m->scale, m->max_kv, m->scores,
                                             nullptr, nullptr, m->attn, st);
        } else if (m->fused_attn) {
            // with the O projection's weight tiles and the MoE router's
            // rows read into L2 alongside, each on the XCD of the workgroup
            // that reads them next (O: workgroup t per 16-row tile; the
            // MoE decode's chain workgroup b: router rows 4b .. 4b + 3)
            const size_t o_tile = (size_t)(qdim / 256) * 16 * 210;  // 16 rows x 210 B per block
            const int n_router = llamd::moe_router_rows(l.moe);
            const float *router = llamd::moe_router(l.moe);
            rc |= llamd::launch_attend_fused(
                m->q, m->k, m->v, l.q_norm, l.k_norm, m->rope, m->tokpos + 1, m->n_head,
                m->n_head_kv, m->hd, m->eps, m->scale, m->max_kv, l.kc, l.vc, m->aq, m->ad, nullptr,
                st, m->prefetch ? l.attn_out : nullptr, o_tile, m->prefetch ? (E + 15) / 16 : 0,
                m->prefetch && router ? router : nullptr, (size_t)4 * E * 4,
                m->prefetch && router ? (n_router + 3) / 4 : 0);
        } else {
            rc |= llamd::launch_qk_norm_rope_store(m->q, m->k, m->v, l.q_norm, l.k_norm, m->rope,
                                                   m->tokpos + 1, m->n_head, m->n_head_kv, m->hd,
                                                   m->eps, l.kc, l.vc, st);
            rc |= llamd::launch_attend_decode(m->q, l.kc, l.vc, m->tokpos + 1, m->n_head,
                                              m->n_head_kv, m->hd, m->scale, m->attn, st);
            llamd_fwd_quantize(m->attn, m->aq, m->ad, qdim / 256);
        }
        // O projection (from the f32 attention output after the split
        // attention: its Q8_K formed inside the matvec)
        if (long_ctx) rc |= llamd::launch_q6k_mv_f32x(l.attn_out, m->attn, m->o, E, qdim / 256, st);
        else llamd_fwd_matvec(l.attn_out, m->aq, m->ad, m->o, qdim / 256, E);
        // ffn_inp = x + O, ffn_norm; then the MoE FFN with the second
        // residual: x = ffn_inp + moe
        if (m->fused_norm) {
            rc |= llamd::moe_forward_normed(l.moe, m->x, m->o, l.ffn_norm, m->eps, m->ffn_inp, m->x);
        } else {
            rc |= llamd::launch_add_rms_norm_mul(m->x, m->o, l.ffn_norm, m->ffn_inp, m->fn, E,
                                                 m->eps, st);
            rc |= llamd_hip_moe_forward(l.moe, m->fn, m->ffn_inp, m->x, 0);
        }
    }
    if (rc || llamd_fwd_last_error()) return set_error("model: a launch failed (%s)", llamd_hip_last_error()) == 0;
    // output norm and the LM head's Q8_K in one launch (the bits of
    // rms_norm * w followed by quantize_q8_k), then matvec + arg-max
    llamd_fwd_rms_norm_quant(m->x, m->output_norm, nullptr, m->aq, m->ad, m->inv, E, m->eps);
    return llamd::lmhead_forward_q8k(m->lmhead, m->aq, m->ad, m->logits, m->next) == 0;
}

void destroy(Model *m) {
    if (!m) return;
    (void)llamd_fwd_sync();
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->exec_long) (void)hipGraphExecDestroy(m->exec_long);
    if (m->lmhead) llamd_hip_lmhead_destroy(m->lmhead);
    for (Layer &l : m->layers) {
        if (l.moe) llamd_hip_moe_destroy(l.moe);
        for (void *w : {l.attn_q, l.attn_k, l.attn_v, l.attn_out})
            if (w) llamd_rocm_release(w);
    }
    if (m->output && m->output_owned) llamd_rocm_release(m->output);
    if (m->tok_embd) llamd_rocm_release(m->tok_embd);
    for (void *p : m->owned) llamd_fwd_free(p);
    if (m->stage) (void)hipHostFree(m->stage);
    delete m;
}

}  // namespace

extern "C" {

void *llamd_hip_model_create(void *g, int max_kv) {
    if (!g || max_kv <= 0) { set_error("model: bad arguments"); return nullptr; }
    if (max_kv > llamd::attend_max_kv()) { set_error("model: max_kv %d above %d", max_kv, llamd::attend_max_kv()); return nullptr; }
    if (llamd_fwd_stream_init()) return nullptr;
    // hyperparameters (crates/llamd-models/src/hparams.rs:77-135)
    const int64_t ai = llamd_gguf_find_kv(g, "general.architecture");
    if (ai < 0) { set_error("hparams: general.architecture is absent"); return nullptr; }
    char arch[64];
    uint64_t alen;
    if (llamd_gguf_kv_str(g, (uint64_t)ai, 0, arch, sizeof arch, &alen)) return nullptr;
    if (strcmp(arch, "qwen3moe") != 0) { set_error("architecture: %s; this device model implements qwen3moe", arch); return nullptr; }
    const std::string p = arch;
    uint64_t n_layer, n_embd, n_head, n_head_kv, hd = 0;
    float eps, base;
    if (!get_u(g, p + ".block_count", &n_layer) || !get_u(g, p + ".embedding_length", &n_embd) ||
        !get_u(g, p + ".attention.head_count", &n_head) ||
        !get_u(g, p + ".attention.head_count_kv", &n_head_kv)) {
        set_error("hparams: a block_count / embedding_length / head_count key is absent");
        return nullptr;
    }
    if (llamd_gguf_get_f32(g, (p + ".attention.layer_norm_rms_epsilon").c_str(), &eps) ||
        llamd_gguf_get_f32(g, (p + ".rope.freq_base").c_str(), &base)) {
        set_error("hparams: rms epsilon or rope.freq_base is absent");
        return nullptr;
    }
    if (!get_u(g, p + ".attention.key_length", &hd)) {
        // the attn_k tensor decides (hparams.rs:100-113)
        const int64_t ki = llamd_gguf_find_tensor(g, "blk.0.attn_k.weight");
        uint32_t nd, type;
        uint64_t dims[4], off;
        if (ki >= 0 && !llamd_gguf_tensor(g, (uint64_t)ki, nullptr, 0, &nd, dims, &type, &off) && n_head_kv)
            hd = dims[1] / n_head_kv;
        else
            hd = n_head ? n_embd / n_head : 0;
    }
    const int64_t ei = llamd_gguf_find_tensor(g, "token_embd.weight");
    if (ei < 0) { set_error("hparams: token_embd.weight is absent"); return nullptr; }
    uint32_t nd, etype;
    uint64_t edims[4], off;
    if (llamd_gguf_tensor(g, (uint64_t)ei, nullptr, 0, &nd, edims, &etype, &off)) return nullptr;
    if (n_head_kv == 0 || n_head % n_head_kv || hd % 2 || hd == 0 || hd > 256 || n_embd % 256 ||
        (n_head * hd) % 256 || n_layer == 0 || n_layer > 4096) {
        set_error("hparams: unsupported shape (n_embd %llu, heads %llu/%llu, head_dim %llu)",
                  (unsigned long long)n_embd, (unsigned long long)n_head,
                  (unsigned long long)n_head_kv, (unsigned long long)hd);
        return nullptr;
    }
    if (etype != 14 || edims[0] != n_embd) { set_error("model: token_embd.weight must be Q6_K [n_embd, n_vocab]"); return nullptr; }

    Model *m = new Model();
    m->n_layer = (int)n_layer;
    m->n_embd = (int)n_embd;
    m->n_head = (int)n_head;
    m->n_head_kv = (int)n_head_kv;
    m->hd = (int)hd;
    m->n_vocab = (int)edims[1];
    m->max_kv = max_kv;
    m->use_graph = llamd::g_tune_model_graph != 0;
    m->fused_norm = llamd::g_tune_model_fused_norm != 0;
    m->norm_qkv = llamd::g_tune_model_norm_qkv != 0;
    m->prefetch = llamd::g_tune_model_prefetch != 0;
    m->fused_attn = llamd::g_tune_model_fused_attn != 0 &&
                    llamd::attend_fused_prepare((int)n_head, (int)n_head_kv, (int)hd, max_kv) == 0;
    m->long_from = llamd::g_tune_model_long_from;
    m->split_attn = m->long_from >= 0 && m->long_from < max_kv &&
                    (int)(n_head * hd) / 256 <= 16 &&  // the f32-input O matvec (launch_q6k_mv_f32x)
                    llamd::attend_split_prepare((int)n_head, (int)n_head_kv, (int)hd, max_kv) == 0;
    m->eps = eps;
    m->rope_base = base;
    m->scale = 1.0f / sqrtf((float)hd);  // attention.rs:95
    const int kv_dim = m->n_head_kv * m->hd, qdim = m->n_head * m->hd;
    bool ok = true;
    auto fail_out = [&](void) -> void * { destroy(m); return nullptr; };

    // embedding table (raw, for row lookups) and the output projection
    {
        uint64_t nb;
        const void *src = llamd_gguf_tensor_data(g, (uint64_t)ei, &nb);
        m->tok_embd = src ? llamd_rocm_upload(src, nb) : nullptr;
        if (!m->tok_embd) return fail_out();
    }
    if (llamd_gguf_find_tensor(g, "output.weight") >= 0) {
        m->output = llamd_gguf_upload_q6k(g, "output.weight");
        m->output_owned = true;
    } else {
        m->output = llamd_gguf_upload_q6k(g, "token_embd.weight");  // tied (layer.rs:295-302)
        m->output_owned = true;
    }
    if (!m->output) return fail_out();
    m->output_norm = upload_f32(*m, g, "output_norm.weight", n_embd);
    if (!m->output_norm) return fail_out();
    m->lmhead = llamd_hip_lmhead_create(m->output, m->n_vocab, m->n_embd / 256, 1);
    if (!m->lmhead) return fail_out();

    m->layers.resize(m->n_layer);
    for (int il = 0; il < m->n_layer && ok; ++il) {
        Layer &l = m->layers[il];
        const std::string b = "blk." + std::to_string(il) + ".";
        l.attn_norm = upload_f32(*m, g, b + "attn_norm.weight", n_embd);
        l.ffn_norm = l.attn_norm ? upload_f32(*m, g, b + "ffn_norm.weight", n_embd) : nullptr;
        l.attn_q = l.ffn_norm ? llamd_gguf_upload_q6k(g, (b + "attn_q.weight").c_str()) : nullptr;
        l.attn_k = l.attn_q ? llamd_gguf_upload_q6k(g, (b + "attn_k.weight").c_str()) : nullptr;
        l.attn_v = l.attn_k ? llamd_gguf_upload_q6k(g, (b + "attn_v.weight").c_str()) : nullptr;
        l.attn_out = l.attn_v ? llamd_gguf_upload_q6k(g, (b + "attn_output.weight").c_str()) : nullptr;
        ok = l.attn_out != nullptr;
        if (ok && llamd_gguf_find_tensor(g, (b + "attn_q_norm.weight").c_str()) >= 0) {
            l.q_norm = upload_f32(*m, g, b + "attn_q_norm.weight", hd);
            ok = l.q_norm != nullptr;
        }
        if (ok && llamd_gguf_find_tensor(g, (b + "attn_k_norm.weight").c_str()) >= 0) {
            l.k_norm = upload_f32(*m, g, b + "attn_k_norm.weight", hd);
            ok = l.k_norm != nullptr;
        }
        if (ok) {
            l.moe = llamd_gguf_moe_create(g, il);
            ok = l.moe != nullptr;
        }
        if (ok) {
            l.kc = dalloc(*m, (size_t)max_kv * kv_dim * 4);
            l.vc = dalloc(*m, (size_t)max_kv * kv_dim * 4);
            ok = l.kc && l.vc;
        }
    }
    if (!ok) return fail_out();
    // the FFN norm inside the MoE decode launch, when the layer's shapes allow it
    // (decided once here: a launch error in the step is then always an error)
    m->fused_norm = m->fused_norm && llamd::moe_normed_applies(m->layers[0].moe);
    {
        const int rows[3] = {qdim, kv_dim, kv_dim};
        m->norm_qkv = m->norm_qkv && llamd::norm_qkv_fits(n_embd, rows);
    }

    // RoPE table: theta = pos / powf(base, 2i/hd), sin / cos (llamd-cpu lib.rs:196-200),
    // with the host libm the reference's f32 powf / sin / cos call
    {
        const int half = m->hd / 2;
        std::vector<float2> cs((size_t)max_kv * half);
        for (int pos = 0; pos < max_kv; ++pos) {
            const float pf = (float)pos * 1.0f;
            for (int i = 0; i < half; ++i) {
                const float exponent = 2.0f * (float)i / (float)m->hd;
                const float theta = pf / powf(base, exponent);
                cs[(size_t)pos * half + i] = make_float2(cosf(theta), sinf(theta));
            }
        }
        m->rope = (float2 *)dalloc(*m, cs.size() * sizeof(float2));
        if (!m->rope || llamd_fwd_upload(m->rope, cs.data(), cs.size() * sizeof(float2))) return fail_out();
    }
    // activations
    const size_t E = (size_t)n_embd * 4;
    m->x = dalloc(*m, E);
    m->xn = dalloc(*m, E);
    m->ffn_inp = dalloc(*m, E);
    m->fn = dalloc(*m, E);
    m->o = dalloc(*m, E);
    m->q = dalloc(*m, (size_t)qdim * 4);
    m->attn = dalloc(*m, (size_t)qdim * 4);
    m->k = dalloc(*m, (size_t)kv_dim * 4);
    m->v = dalloc(*m, (size_t)kv_dim * 4);
    const size_t maxk = qdim > m->n_embd ? qdim : m->n_embd;
    m->aq = (int8_t *)dalloc(*m, maxk);
    m->ad = dalloc(*m, maxk / 256 * 4);
    m->inv = dalloc(*m, 16);
    m->logits = dalloc(*m, (size_t)m->n_vocab * 4);
    m->tokpos = (int32_t *)dalloc(*m, 16);
    m->next = (int32_t *)dalloc(*m, 16);
    if (m->split_attn) {
        m->scores = dalloc(*m, (size_t)m->n_head * max_kv * 4);
        if (!m->scores) m->split_attn = false;
    }
    if (hipHostMalloc((void **)&m->stage, 64, hipHostMallocDefault) != hipSuccess) m->stage = nullptr;
    if (!m->x || !m->xn || !m->ffn_inp || !m->fn || !m->o || !m->q || !m->attn || !m->k || !m->v ||
        !m->aq || !m->ad || !m->inv || !m->logits || !m->tokpos || !m->next || !m->stage) {
        set_error("model: activation buffers could not be allocated");
        return fail_out();
    }
    if (llamd_fwd_sync()) return fail_out();
    return m;
}

void llamd_hip_model_destroy(void *h) { destroy((Model *)h); }

int llamd_hip_model_info(void *h, int *n_layer, int *n_embd, int *n_vocab, int *max_kv) {
    const Model *m = (const Model *)h;
    if (!m) return set_error("model: null handle");
    if (n_layer) *n_layer = m->n_layer;
    if (n_embd) *n_embd = m->n_embd;
    if (n_vocab) *n_vocab = m->n_vocab;
    if (max_kv) *max_kv = m->max_kv;
    return 0;
}

int llamd_hip_model_forward(void *h, int token, int pos, float *logits, int32_t *next) {
    Model *m = (Model *)h;
    if (!m) return set_error("model: null handle");
    if (token < 0 || token >= m->n_vocab) return set_error("model: token %d outside a vocabulary of %d", token, m->n_vocab);
    if (pos < 0 || pos >= m->max_kv) return set_error("model: position %d beyond the %d allocated", pos, m->max_kv);
    hipStream_t st = (hipStream_t)llamd_fwd_get_stream();
    // token and position through the page-locked stage: an asynchronous
    // copy (the stage is rewritten only after the previous call's sync)
    m->stage[0] = token;
    m->stage[1] = pos;
    if (hipMemcpyAsync(m->tokpos, m->stage, 8, hipMemcpyHostToDevice, st) != hipSuccess)
        return set_error("model: token upload failed");
    // The step reads token and position from device memory, so its launches
    // are the same for every token: captured once into a HIP graph, replayed
    // per token (no per-launch host work). If capture is refused, the step
    // runs as plain launches.
    // positions from long_from on take the split attention (its own graph)
    const bool long_ctx = m->split_attn && pos >= m->long_from;
    hipGraphExec_t &exec = long_ctx ? m->exec_long : m->exec;
    if (!exec && m->use_graph) {
        hipGraph_t graph = nullptr;
        bool ok = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) == hipSuccess;
        const bool enq = ok && enqueue_step(m, st, long_ctx);
        ok = hipStreamEndCapture(st, &graph) == hipSuccess && ok && enq;
        ok = ok && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
        if (graph) (void)hipGraphDestroy(graph);
        if (!ok) {
            exec = nullptr;
            m->use_graph = false;
            (void)hipGetLastError();
        }
    }
    if (exec) {
        if (hipGraphLaunch(exec, st) != hipSuccess) return set_error("model: graph launch failed");
    } else if (!enqueue_step(m, st, long_ctx)) {
        return -1;
    }
    // both results queued, then one synchronisation (logits straight into
    // the caller's buffer: one DMA when it is page-locked)
    if (logits && hipMemcpyAsync(logits, m->logits, (size_t)m->n_vocab * 4, hipMemcpyDeviceToHost,
                                 st) != hipSuccess)
        return set_error("model: logits download failed");
    if (hipMemcpyAsync(m->stage + 2, m->next, 4, hipMemcpyDeviceToHost, st) != hipSuccess)
        return set_error("model: download failed");
    if (hipStreamSynchronize(st) != hipSuccess) return set_error("model: step failed");
    if (next) *next = m->stage[2];
    return 0;
}

}  // extern "C"
