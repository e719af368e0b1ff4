// capi.cpp -- the C ABI declared in include/llamd_hip.h.
//
// Host-side C++: argument validation, device memory, the library stream, and
// the MoE-layer / LM-head handles that queue the gfx950 kernels of
// q6k_mv.hip, q8k.hip, moe.hip and group.hip. Validation happens here, before
// any launch, so a bad shape or expert id is an error return and never an
// out-of-bounds device access (the reference does the same checks in its Rust
// wrappers, crates/llamd-rocm/src/lib.rs:434-470).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/llamd_hip.h"
#include "errors.hpp"
#include "launch.hpp"

using namespace llamd;

namespace {

constexpr int QK = 256;
constexpr int SEGB = 16 * 210;

thread_local char g_err[512] = "";
// Set by a device-pointer launcher (void in the reference's ABI) that refused
// its arguments; llamd_fwd_last_error reports it once, then clears it.
bool g_fwd_refused = false;
std::mutex g_mu;             // serialises host-in/host-out calls and the registry
hipStream_t g_stream = nullptr;
// MoE decode schedule: 2 router fold beside gate/up, then down (moe_decode.hip);
// 1 router, gate/up + SwiGLU, down + combine; 0 unfused (separate SwiGLU).
// batched decode: up to this many sequences through the decode kernels, more
// through the expert-grouped (prefill) kernels. Measured on MI355X (configs[2]
// layer, us per token, decode / grouped): 12 sequences 9.06 / 9.31, 16
// sequences 8.89 / 8.05.
int g_tune_batch_decode_max = 12;
// loads per cross-workgroup wait in the MoE decode kernel before the waiting
// wave computes the value itself (0: always)
int g_tune_moe_polls = 1 << 18;
}  // namespace
int llamd::g_tune_model_graph = 1;  // whole-token decode replays a captured graph
int llamd::g_tune_model_fused_attn = 1;  // decode step: attend_fused (else three launches)
int llamd::g_tune_model_fused_norm = 1;  // decode step: FFN norm inside the MoE decode launch
int llamd::g_tune_model_norm_qkv = 1;  // decode step: attention norm inside the Q/K/V launch
int llamd::g_tune_model_prefetch = 1;  // decode step: O weights into L2 under the attention
int llamd::g_tune_model_long_from = 256;  // decode step: split attention from this position (-1: never)
namespace {

int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

}  // namespace

void llamd::fwd_refused() { g_fwd_refused = true; }

namespace {
// A void launcher's launch: a refusal (the launcher's -1) or a failed launch
// is recorded for llamd_fwd_last_error, with the reason.
void checked(int rc, const char *what) {
    if (rc) {
        fail("%s: arguments refused or launch failed", what);
        llamd::fwd_refused();
    }
}
}  // namespace

// The error text of the calling thread, for the other host files of the
// library (errors.hpp).
int llamd::set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

namespace {

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    fail("%s: %s", what, hipGetErrorString(e));
    return false;
}

hipStream_t stream() {
    if (!g_stream) {
        if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) g_stream = nullptr;
    }
    return g_stream;
}

// Registry of uploaded weights so that every entry point can check that a
// handle is what it claims and that its shape covers the request.
enum Kind { KIND_Q6K = 1, KIND_Q8_0 = 2 };
struct WInfo {
    Kind kind;
    int rows;        // rows per expert matrix
    int blocks;      // 256-blocks per row (Q6_K) or k (Q8_0)
    int n_expert;    // matrices in the upload
    size_t stride;   // bytes between expert matrices
};
std::unordered_map<const void *, WInfo> g_weights;

bool lookup(const void *p, Kind kind, WInfo *out) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_weights.find(p);
    if (it == g_weights.end() || it->second.kind != kind) return false;
    *out = it->second;
    return true;
}

struct DevBuf {
    void *p = nullptr;
    DevBuf() = default;
    explicit DevBuf(size_t n) { alloc(n); }
    bool alloc(size_t n) {
        release();
        if (n == 0) n = 16;
        if (hipMalloc(&p, n) != hipSuccess) p = nullptr;
        return p != nullptr;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
    }
    ~DevBuf() { release(); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    template <class T> T *as() const { return (T *)p; }
};

bool up(void *dst, const void *src, size_t n) {
    return hip_ok(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, stream()), "upload");
}
bool down(void *dst, const void *src, size_t n) {
    return hip_ok(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, stream()), "download");
}
bool sync() { return hip_ok(hipStreamSynchronize(stream()), "synchronize"); }

int quantize_dev(const float *d_x, int8_t *d_qs, float *d_d, int16_t *d_bs, int nblocks) {
    return launch_q8k_quantize(d_x, d_qs, d_d, d_bs, nblocks, stream());
}

constexpr int CHUNK = 16;             // tokens per chunk of the batched operand layout
constexpr size_t CHUNK_BLOCK = 4096;  // bytes per (chunk, block)

size_t chunk_q_bytes(int nseq, int blocks) {
    return (size_t)((nseq + CHUNK - 1) / CHUNK) * blocks * CHUNK_BLOCK;
}
size_t chunk_d_bytes(int nseq, int blocks) {
    return (size_t)((nseq + CHUNK - 1) / CHUNK) * blocks * CHUNK * 4;
}

// Single-group batched matvec: all rows, nseq tokens in chunk slots 0..nseq-1.
int batched_dev(const void *w, const int8_t *cq, const float *cd, float *y, int blocks, int rows,
                int nseq) {
    return launch_q6k_mv_batched(w, 0, nullptr, nullptr, nullptr, nullptr, nullptr, cq, cd, y, rows,
                                 rows, blocks, nseq, (nseq + CHUNK - 1) / CHUNK, stream());
}

}  // namespace

// Resolve a Q6_K weight pointer to the tiled layout the kernels read
// (launch.hpp Q6kView). Tiled uploads (llamd_rocm_upload_q6k[_experts]) are
// used as they are. Anything else is the reference's own device layout --
// ggml blocks (planar_off null) or the planar repack -- in memory from
// llamd_fwd_alloc / llamd_rocm_upload, and resolves to its tiled copy
// (compat_abi.cpp). grouped: `rows` per expert of an expert tensor, either one
// upload of rows*n rows (rows % 16 == 0) or llamd_rocm_upload_q6k_experts;
// otherwise a matrix of at least `rows` rows.
int llamd::resolve_q6k(const void *d_w, const size_t *planar_off, int rows, int blocks,
                       bool grouped, Q6kView *v) {
    if (!d_w) return fail("Q6_K weight: null pointer");
    if (rows <= 0 || blocks <= 0) return fail("Q6_K weight: rows %d, blocks %d", rows, blocks);
    WInfo wi;
    int total = 0;
    if (!planar_off && lookup(d_w, KIND_Q6K, &wi)) {
        if (blocks != wi.blocks) return fail("blocks %d != uploaded %d", blocks, wi.blocks);
        v->tiled = d_w;
        if (wi.n_expert > 1) {
            if (grouped ? rows != wi.rows : rows > wi.rows)
                return fail("rows %d do not match the uploaded expert rows %d", rows, wi.rows);
            v->expert_stride = wi.stride;
            v->n_expert = wi.n_expert;
            return 0;
        }
        total = wi.rows;
    } else {
        if (shadow_q6k(d_w, planar_off, rows, blocks, &v->tiled, &total)) return -1;
    }
    if (!grouped) {
        if (rows > total) return fail("rows %d exceed the weight's %d", rows, total);
        v->expert_stride = 0;
        v->n_expert = 1;
        return 0;
    }
    if (total % rows) return fail("rows %d does not divide the weight's %d", rows, total);
    if (total != rows && rows % 16) return fail("rows %d not a multiple of 16", rows);
    v->expert_stride = (size_t)(rows / 16) * blocks * SEGB;
    v->n_expert = total / rows;
    return 0;
}

static int expert_view(const void *d_w, int rows, int blocks, size_t *stride, int *n_expert,
                       const void **tiled) {
    Q6kView v;
    if (resolve_q6k(d_w, nullptr, rows, blocks, true, &v)) return -1;
    *stride = v.expert_stride;
    *n_expert = v.n_expert;
    *tiled = v.tiled;
    return 0;
}


extern "C" {

const char *llamd_hip_last_error(void) { return g_err; }

int llamd_hip_tune(const char *key, int value) {
    if (!key) return fail("tune: null key");
    if (!strcmp(key, "model_fused_norm")) {
        const int prev = g_tune_model_fused_norm;
        g_tune_model_fused_norm = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "model_norm_qkv")) {
        const int prev = g_tune_model_norm_qkv;
        g_tune_model_norm_qkv = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "model_prefetch")) {
        const int prev = g_tune_model_prefetch;
        g_tune_model_prefetch = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "model_long_from")) {
        const int prev = g_tune_model_long_from;
        g_tune_model_long_from = value;
        return prev;
    }
    if (!strcmp(key, "model_fused_attn")) {
        const int prev = g_tune_model_fused_attn;
        g_tune_model_fused_attn = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "model_graph")) {
        const int prev = g_tune_model_graph;
        g_tune_model_graph = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "moe_polls")) {
        const int prev = g_tune_moe_polls;
        g_tune_moe_polls = value < 0 ? 0 : value;
        return prev;
    }
    if (!strcmp(key, "batch_decode_max")) {
        const int prev = g_tune_batch_decode_max;
        g_tune_batch_decode_max = value;
        return prev;
    }
    if (!strcmp(key, "batched_twin")) {
        const int prev = g_tune_batched_twin;
        g_tune_batched_twin = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "fast_lds")) {
        const int prev = g_tune_fast_lds;
        g_tune_fast_lds = value ? 1 : 0;
        return prev;
    }
    if (!strcmp(key, "fast_ks")) {
        if (value != 0 && value != 1 && value != 2 && value != 4)
            return fail("tune: fast_ks takes 0 (by shape), 1, 2 or 4");
        const int prev = g_tune_fast_ks;
        g_tune_fast_ks = value;
        return prev;
    }
    if (!strcmp(key, "mv_ks")) {
        if (value != 0 && value != 1 && value != 4 && value != 8)
            return fail("tune: mv_ks takes 0 (by shape), 1, 4 or 8");
        const int prev = g_tune_mv_ks;
        g_tune_mv_ks = value;
        return prev;
    }
    return fail("tune: unknown key %s", key);
}

// ---- inventory ---------------------------------------------------------------
int llamd_rocm_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int llamd_rocm_device_info(int dev, char *name, int name_len, char *arch, int arch_len,
                           size_t *total_mem, int *wgp_count, int *warp_size) {
    hipDeviceProp_t p;
    if (!hip_ok(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties")) return -1;
    if (name && name_len > 0) snprintf(name, name_len, "%s", p.name);
    if (arch && arch_len > 0) snprintf(arch, arch_len, "%s", p.gcnArchName);
    if (total_mem) *total_mem = p.totalGlobalMem;
    if (wgp_count) *wgp_count = p.multiProcessorCount;
    if (warp_size) *warp_size = p.warpSize;
    return 0;
}

size_t llamd_rocm_free_mem(void) {
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) != hipSuccess) return 0;
    return f;
}

// ---- raw memory / stream -------------------------------------------------------
void *llamd_rocm_upload(const void *host, size_t bytes) {
    if (!host || !bytes) { fail("upload: empty"); return nullptr; }
    void *d = nullptr;
    if (!hip_ok(hipMalloc(&d, bytes), "hipMalloc")) return nullptr;
    if (!hip_ok(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "hipMemcpy")) {
        (void)hipFree(d);
        return nullptr;
    }
    note_alloc(d, bytes);
    return d;
}

void llamd_rocm_release(void *dev) {
    if (!dev) return;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_weights.erase(dev);
    }
    note_free(dev);
    (void)hipFree(dev);
}

// ---- graph capture of the library stream -----------------------------------
// One graph at a time. Capture records launches without running them; the
// first results come from the first replay. Everything the captured calls
// read must be resident (no host copies inside a capture), and no kernel of
// this library records a memset node.
static hipGraph_t g_graph = nullptr;
static hipGraphExec_t g_exec = nullptr;

static void drop_graph() {
    if (g_exec) { (void)hipGraphExecDestroy(g_exec); g_exec = nullptr; }
    if (g_graph) { (void)hipGraphDestroy(g_graph); g_graph = nullptr; }
}

int llamd_fwd_begin_capture(void) {
    if (!stream()) return fail("stream create failed");
    drop_graph();
    // relaxed: a raw or planar Q6_K weight first used inside the capture gets
    // its tiled copy allocated and filled on a side stream (compat.hip)
    return hip_ok(hipStreamBeginCapture(stream(), hipStreamCaptureModeRelaxed), "begin capture")
               ? 0 : -1;
}

int llamd_fwd_end_capture(void) {
    if (!stream()) return fail("stream create failed");
    if (!hip_ok(hipStreamEndCapture(stream(), &g_graph), "end capture")) return -1;
    if (!hip_ok(hipGraphInstantiate(&g_exec, g_graph, nullptr, nullptr, 0), "graph instantiate")) {
        drop_graph();
        return -1;
    }
    return 0;
}

int llamd_fwd_graph_launch(void) {
    if (!g_exec) return fail("graph_launch: no graph");
    return hip_ok(hipGraphLaunch(g_exec, stream()), "graph launch") ? 0 : -1;
}

int llamd_fwd_has_graph(void) { return g_exec ? 1 : 0; }

void llamd_fwd_graph_destroy(void) { drop_graph(); }

void *llamd_fwd_get_stream(void) { return (void *)stream(); }
int llamd_fwd_stream_init(void) { return stream() ? 0 : fail("stream create failed"); }

void *llamd_fwd_alloc(size_t bytes) {
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 16), "hipMalloc")) return nullptr;
    note_alloc(p, bytes ? bytes : 16);
    return p;
}
void llamd_fwd_free(void *p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_weights.erase(p);
    }
    note_free(p);
    (void)hipFree(p);
}
int llamd_fwd_upload(void *dst, const void *src, size_t bytes) {
    if (!(up(dst, src, bytes) && sync())) return -1;
    // a tiled copy made of these bytes is re-made from them
    return note_write(dst, bytes, stream()) || !sync() ? -1 : 0;
}
int llamd_fwd_download(void *dst, const void *src, size_t bytes) {
    return down(dst, src, bytes) && sync() ? 0 : -1;
}
int llamd_fwd_sync(void) { return sync() ? 0 : -1; }
int llamd_fwd_last_error(void) {
    if (g_fwd_refused) {
        g_fwd_refused = false;
        return -1;  // g_err holds the refusal
    }
    return hip_ok(hipGetLastError(), "queued work") ? 0 : -1;
}

// ---- weight upload -----------------------------------------------------------
static void *upload_q6k_impl(const void *ggml, int n_expert, int rows, int blocks) {
    if (!ggml || rows <= 0 || blocks <= 0 || n_expert <= 0) {
        fail("upload_q6k: bad shape rows=%d blocks=%d n_expert=%d", rows, blocks, n_expert);
        return nullptr;
    }
    const size_t per = llamd_hip_q6k_tiled_bytes(rows, blocks);
    const size_t ggml_per = (size_t)rows * blocks * 210;
    void *d = nullptr;
    if (!hip_ok(hipMalloc(&d, per * n_expert), "hipMalloc")) return nullptr;
    std::vector<uint8_t> tmp(per);
    for (int e = 0; e < n_expert; ++e) {
        llamd_hip_q6k_tile((const uint8_t *)ggml + e * ggml_per, rows, blocks, tmp.data());
        if (!hip_ok(hipMemcpy((uint8_t *)d + e * per, tmp.data(), per, hipMemcpyHostToDevice),
                    "hipMemcpy")) {
            (void)hipFree(d);
            return nullptr;
        }
    }
    std::lock_guard<std::mutex> lk(g_mu);
    g_weights[d] = WInfo{KIND_Q6K, rows, blocks, n_expert, per};
    return d;
}

void *llamd_rocm_upload_q6k(const void *ggml, int rows, int blocks) {
    return upload_q6k_impl(ggml, 1, rows, blocks);
}

void *llamd_rocm_upload_q6k_experts(const void *ggml, int n_expert, int rows, int blocks) {
    return upload_q6k_impl(ggml, n_expert, rows, blocks);
}

void *llamd_hip_upload_q8_0(const void *ggml, int rows, int k) {
    const size_t bytes = llamd_hip_q8_0_planar_bytes(rows, k);
    if (!ggml || !bytes) {
        fail("upload_q8_0: bad shape rows=%d k=%d", rows, k);
        return nullptr;
    }
    std::vector<uint8_t> tmp(bytes);
    llamd_hip_q8_0_planarize(ggml, rows, k, tmp.data());
    void *d = llamd_rocm_upload(tmp.data(), bytes);
    if (!d) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    g_weights[d] = WInfo{KIND_Q8_0, rows, k, 1, bytes};
    return d;
}

// ---- host-in/host-out ----------------------------------------------------------
int llamd_rocm_matvec_q6k_resident(const void *d_w, const int8_t *aq, const float *ad, float *out,
                                   int blocks, int rows) {
    if (!aq || !ad || !out) return fail("matvec: null pointer");
    Q6kView v;
    if (resolve_q6k(d_w, nullptr, rows, blocks, false, &v)) return -1;
    d_w = v.tiled;
    std::lock_guard<std::mutex> lk(g_mu);
    DevBuf q((size_t)blocks * QK), d((size_t)blocks * 4), y((size_t)rows * 4);
    if (!q.p || !d.p || !y.p) return fail("hipMalloc");
    if (!up(q.p, aq, (size_t)blocks * QK) || !up(d.p, ad, (size_t)blocks * 4)) return -1;
    if (launch_q6k_mv_b1(d_w, 0, nullptr, q.as<int8_t>(), d.as<float>(), y.as<float>(), rows,
                         blocks, 1, 0, stream()))
        return fail("launch");
    if (!down(out, y.p, (size_t)rows * 4) || !sync()) return -1;
    return 0;
}

static int grouped_host(const void *d_w, const int32_t *eid, const int8_t *aq, const float *ad,
                        float *out, int blocks, int rows, int n_used, int per_slot) {
    if (n_used <= 0) return fail("grouped: no experts");
    if (!eid || !aq || !ad || !out) return fail("grouped: null pointer");
    size_t stride = 0;
    int n_expert = 0;
    if (expert_view(d_w, rows, blocks, &stride, &n_expert, &d_w)) return -1;
    for (int i = 0; i < n_used; ++i)
        if (eid[i] < 0 || eid[i] >= n_expert)
            return fail("grouped: expert id %d out of range [0,%d)", eid[i], n_expert);
    std::lock_guard<std::mutex> lk(g_mu);
    const int n_act = per_slot ? n_used : 1;
    DevBuf q((size_t)n_act * blocks * QK), d((size_t)n_act * blocks * 4),
        y((size_t)rows * n_used * 4), ids((size_t)n_used * 4);
    if (!q.p || !d.p || !y.p || !ids.p) return fail("hipMalloc");
    if (!up(q.p, aq, (size_t)n_act * blocks * QK) || !up(d.p, ad, (size_t)n_act * blocks * 4) ||
        !up(ids.p, eid, (size_t)n_used * 4))
        return -1;
    if (launch_q6k_mv_b1(d_w, stride, ids.as<int32_t>(), q.as<int8_t>(), d.as<float>(),
                         y.as<float>(), rows, blocks, n_used, per_slot, stream()))
        return fail("launch");
    if (!down(out, y.p, (size_t)rows * n_used * 4) || !sync()) return -1;
    return 0;
}

int llamd_rocm_matvec_grouped(const void *d_w, const int32_t *eid, const int8_t *aq,
                              const float *ad, float *out, int blocks, int rows, int n_used) {
    return grouped_host(d_w, eid, aq, ad, out, blocks, rows, n_used, 0);
}

int llamd_hip_matvec_grouped_pa(const void *d_w, const int32_t *eid, const int8_t *aq,
                                const float *ad, float *out, int blocks, int rows, int n_used) {
    return grouped_host(d_w, eid, aq, ad, out, blocks, rows, n_used, 1);
}

// Batched host entry: quantized activations given in natural order; they are
// re-ordered class-major on the host for the kernel's operand loads.
int llamd_hip_matvec_q6k_batched(const void *d_w, const int8_t *aq, const float *ad, float *out,
                                 int blocks, int rows, int nseq) {
    if (nseq <= 0 || !aq || !ad || !out) return fail("batched: bad arguments");
    Q6kView v;
    if (resolve_q6k(d_w, nullptr, rows, blocks, false, &v)) return -1;
    d_w = v.tiled;
    // the reference's BlockQ8K arrays -> the token-chunked operand layout
    const size_t nq = chunk_q_bytes(nseq, blocks), nd = chunk_d_bytes(nseq, blocks);
    std::vector<int8_t> cq(nq, 0);
    std::vector<float> cd(nd / 4, 0.0f);
    for (int t = 0; t < nseq; ++t)
        for (int b = 0; b < blocks; ++b) {
            const size_t base = (size_t)(t / CHUNK) * blocks + b;
            for (int e = 0; e < QK; ++e)
                cq[base * CHUNK_BLOCK + (e % 8) * 512 + (t % CHUNK) * 32 + e / 8] =
                    aq[((size_t)t * blocks + b) * QK + e];
            cd[base * CHUNK + t % CHUNK] = ad[(size_t)t * blocks + b];
        }
    std::lock_guard<std::mutex> lk(g_mu);
    DevBuf q(nq), d(nd), y((size_t)rows * nseq * 4);
    if (!q.p || !d.p || !y.p) return fail("hipMalloc");
    if (!up(q.p, cq.data(), nq) || !up(d.p, cd.data(), nd)) return -1;
    if (batched_dev(d_w, q.as<int8_t>(), d.as<float>(), y.as<float>(), blocks, rows, nseq))
        return fail("launch");
    if (!down(out, y.p, (size_t)rows * nseq * 4) || !sync()) return -1;
    return 0;
}

int llamd_rocm_quantize_q8k(const float *x, int nblocks, int8_t *qs, float *d, int16_t *bsums) {
    if (nblocks <= 0 || !x || !qs || !d) return fail("quantize: bad arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    DevBuf dx((size_t)nblocks * QK * 4), dq((size_t)nblocks * QK), dd((size_t)nblocks * 4),
        db((size_t)nblocks * 32);
    if (!dx.p || !dq.p || !dd.p || !db.p) return fail("hipMalloc");
    if (!up(dx.p, x, (size_t)nblocks * QK * 4)) return -1;
    if (quantize_dev(dx.as<float>(), dq.as<int8_t>(), dd.as<float>(), db.as<int16_t>(),
                     nblocks))
        return fail("launch");
    if (!down(qs, dq.p, (size_t)nblocks * QK) || !down(d, dd.p, (size_t)nblocks * 4)) return -1;
    if (bsums && !down(bsums, db.p, (size_t)nblocks * 32)) return -1;
    return sync() ? 0 : -1;
}

int llamd_hip_swiglu_q8k(const float *gate, const float *upv, int nblocks, float *act, int8_t *qs,
                         float *d, int16_t *bsums) {
    if (nblocks <= 0 || !gate || !upv || !qs || !d) return fail("swiglu: bad arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t n = (size_t)nblocks * QK;
    DevBuf dg(n * 4), du(n * 4), da(n * 4), dq(n), dd((size_t)nblocks * 4), db((size_t)nblocks * 32);
    if (!dg.p || !du.p || !da.p || !dq.p || !dd.p || !db.p) return fail("hipMalloc");
    if (!up(dg.p, gate, n * 4) || !up(du.p, upv, n * 4)) return -1;
    if (launch_swiglu_q8k(dg.as<float>(), du.as<float>(), da.as<float>(), dq.as<int8_t>(),
                          dd.as<float>(), db.as<int16_t>(), nblocks, stream()))
        return fail("launch");
    if (act && !down(act, da.p, n * 4)) return -1;
    if (!down(qs, dq.p, n) || !down(d, dd.p, (size_t)nblocks * 4)) return -1;
    if (bsums && !down(bsums, db.p, (size_t)nblocks * 32)) return -1;
    return sync() ? 0 : -1;
}

int llamd_hip_dequant_q6k(const void *d_w, int rows, int blocks, float *out) {
    if (!out) return fail("dequant: null output");
    WInfo wi;
    if (lookup(d_w, KIND_Q6K, &wi) && (wi.n_expert != 1 || rows != wi.rows || blocks != wi.blocks))
        return fail("dequant: shape mismatch");
    // a raw ggml tensor dequantizes through its tiled copy (its first rows rows)
    Q6kView v;
    if (resolve_q6k(d_w, nullptr, rows, blocks, false, &v)) return -1;
    d_w = v.tiled;
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t n = (size_t)rows * blocks * QK;
    DevBuf y(n * 4);
    if (!y.p) return fail("hipMalloc");
    if (launch_q6k_dequant(d_w, rows, blocks, y.as<float>(), stream())) return fail("launch");
    if (!down(out, y.p, n * 4) || !sync()) return -1;
    return 0;
}

int llamd_hip_dequant_q8_0(const void *d_w, int rows, int k, float *out) {
    WInfo wi;
    if (!lookup(d_w, KIND_Q8_0, &wi)) return fail("not a Q8_0 weight handle");
    if (rows != wi.rows || k != wi.blocks || !out) return fail("dequant: shape mismatch");
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t n = (size_t)rows * k;
    DevBuf y(n * 4);
    if (!y.p) return fail("hipMalloc");
    if (launch_q8_0_dequant(d_w, rows, k, y.as<float>(), stream())) return fail("launch");
    if (!down(out, y.p, n * 4) || !sync()) return -1;
    return 0;
}

int llamd_hip_matvec_q8_0(const void *d_w, const float *x, float *out, int rows, int k) {
    WInfo wi;
    if (!lookup(d_w, KIND_Q8_0, &wi)) return fail("not a Q8_0 weight handle");
    if (rows != wi.rows || k != wi.blocks || !x || !out) return fail("matvec_q8_0: shape mismatch");
    std::lock_guard<std::mutex> lk(g_mu);
    DevBuf dx((size_t)k * 4), y((size_t)rows * 4);
    if (!dx.p || !y.p) return fail("hipMalloc");
    if (!up(dx.p, x, (size_t)k * 4)) return -1;
    if (launch_q8_0_mv(d_w, dx.as<float>(), y.as<float>(), rows, k, stream())) return fail("launch");
    if (!down(out, y.p, (size_t)rows * 4) || !sync()) return -1;
    return 0;
}

int llamd_hip_route(const float *logits, int n_expert, int n_used, int32_t *ids, float *weights) {
    if (!logits || !ids || !weights) return fail("route: null pointer");
    if (n_used <= 0 || n_used > n_expert) return fail("route: %d experts requested of %d", n_used, n_expert);
    if (n_expert > 256 || n_used > 64) return fail("route: at most 256 experts, 64 used");
    std::lock_guard<std::mutex> lk(g_mu);
    DevBuf dl((size_t)n_expert * 4), di((size_t)n_used * 4), dw((size_t)n_used * 4);
    if (!dl.p || !di.p || !dw.p) return fail("hipMalloc");
    if (!up(dl.p, logits, (size_t)n_expert * 4)) return -1;
    if (launch_route_logits(dl.as<float>(), n_expert, n_used, di.as<int32_t>(), dw.as<float>(),
                            stream()))
        return fail("launch");
    if (!down(ids, di.p, (size_t)n_used * 4) || !down(weights, dw.p, (size_t)n_used * 4) || !sync())
        return -1;
    return 0;
}

int llamd_hip_argmax(const float *x, int n, int nseq, int32_t *ids) {
    if (!x || !ids || n <= 0 || nseq <= 0) return fail("argmax: bad arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    const int parts = argmax_parts(n);
    DevBuf dx((size_t)n * nseq * 4), pv((size_t)parts * nseq * 4), pi((size_t)parts * nseq * 4),
        di((size_t)nseq * 4);
    if (!dx.p || !pv.p || !pi.p || !di.p) return fail("hipMalloc");
    if (!up(dx.p, x, (size_t)n * nseq * 4)) return -1;
    if (launch_argmax(dx.as<float>(), n, n, nseq, pv.as<float>(), pi.as<int>(), di.as<int32_t>(),
                      stream()))
        return fail("launch");
    if (!down(ids, di.p, (size_t)nseq * 4) || !sync()) return -1;
    return 0;
}

// ---- device-pointer launchers ------------------------------------------------
void llamd_fwd_matvec(const void *d_w, const int8_t *d_aq, const float *d_ad, float *d_out,
                      int blocks, int rows) {
    Q6kView v;
    if (resolve_q6k(d_w, nullptr, rows, blocks, false, &v)) return fwd_refused();
    if (launch_q6k_mv_b1(v.tiled, 0, nullptr, d_aq, d_ad, d_out, rows, blocks, 1, 0, stream()))
        return (void)fail("matvec: launch"), fwd_refused();
}

void llamd_fwd_matvec_grouped(const void *d_w, const int32_t *d_ids, const int8_t *d_aq,
                              const float *d_ad, float *d_out, int blocks, int rows, int n_used) {
    size_t stride = 0;
    int ne = 0;
    if (n_used <= 0 || expert_view(d_w, rows, blocks, &stride, &ne, &d_w)) return fwd_refused();
    checked(launch_q6k_mv_b1(d_w, stride, d_ids, d_aq, d_ad, d_out, rows, blocks, n_used, 0, stream()),
            "matvec_grouped");
}

void llamd_fwd_matvec_grouped_pa(const void *d_w, const int32_t *d_ids, const int8_t *d_aq,
                                 const float *d_ad, float *d_out, int blocks, int rows,
                                 int n_used) {
    size_t stride = 0;
    int ne = 0;
    if (n_used <= 0 || expert_view(d_w, rows, blocks, &stride, &ne, &d_w)) return fwd_refused();
    checked(launch_q6k_mv_b1(d_w, stride, d_ids, d_aq, d_ad, d_out, rows, blocks, n_used, 1, stream()),
            "matvec_grouped_pa");
}

void llamd_fwd_quantize(const float *d_x, int8_t *d_qs, float *d_d, int nblocks) {
    checked(quantize_dev(d_x, d_qs, d_d, nullptr, nblocks), "quantize");
}

void llamd_fwd_silu_mul(const float *gate, const float *upv, float *out, int n) {
    checked(launch_silu_mul(gate, upv, out, n, stream()), "silu_mul");
}

void llamd_fwd_router(const float *logits, int n_expert, int n_used, int32_t *ids,
                      float *weights, float *probs) {
    if (n_expert <= 0 || n_expert > 256 || n_used <= 0 || n_used > n_expert) {  // route_logits: 4 logits per lane
        fail("router: n_expert %d, n_used %d", n_expert, n_used);
        return fwd_refused();
    }
    checked(launch_route_logits(logits, n_expert, n_used, ids, weights, stream(), 1, probs), "router");
}

void llamd_fwd_matvec_x3(const void *w0, const void *w1, const void *w2, const int8_t *d_aq,
                         const float *d_ad, float *o0, float *o1, float *o2, int blocks, int rows0,
                         int rows1, int rows2) {
    const void *w[3] = {w0, w1, w2};
    float *y[3] = {o0, o1, o2};
    const int rows[3] = {rows0, rows1, rows2};
    for (int i = 0; i < 3; ++i) {
        Q6kView v;
        if (resolve_q6k(w[i], nullptr, rows[i], blocks, false, &v)) return fwd_refused();
        w[i] = v.tiled;
    }
    checked(launch_q6k_mv_x3(w, y, rows, 3, d_aq, d_ad, blocks, stream()), "matvec_x3");
}

void llamd_fwd_matvec_x3_splitk(const void *w0, const void *w1, const void *w2, const int8_t *d_aq,
                                const float *d_ad, float *o0, float *o1, float *o2, int blocks,
                                int rows0, int rows1, int rows2, int nsub) {
    (void)nsub;  // the split of K is chosen by the library
    llamd_fwd_matvec_x3(w0, w1, w2, d_aq, d_ad, o0, o1, o2, blocks, rows0, rows1, rows2);
}

void llamd_fwd_matvec_grouped_x2(const void *wa, const void *wb, const int32_t *d_ids,
                                 const int8_t *d_aq, const float *d_ad, float *oa, float *ob,
                                 int blocks, int rows, int n_used) {
    size_t sa = 0, sb = 0;
    int na = 0, nb = 0;
    if (n_used <= 0 || expert_view(wa, rows, blocks, &sa, &na, &wa) ||
        expert_view(wb, rows, blocks, &sb, &nb, &wb))
        return fwd_refused();
    if (sa != sb) {
        fail("matvec_grouped_x2: the two expert tensors differ in shape");
        return fwd_refused();
    }
    checked(launch_q6k_mv_grouped_x2(wa, wb, sa, d_ids, d_aq, d_ad, oa, ob, rows, blocks, n_used, stream()),
            "matvec_grouped_x2");
}

void llamd_fwd_matvec_grouped_x2_splitk(const void *wa, const void *wb, const int32_t *d_ids,
                                        const int8_t *d_aq, const float *d_ad, float *oa,
                                        float *ob, int blocks, int rows, int n_used, int nsub) {
    (void)nsub;
    llamd_fwd_matvec_grouped_x2(wa, wb, d_ids, d_aq, d_ad, oa, ob, blocks, rows, n_used);
}

void llamd_fwd_matvec_grouped_pa_splitk(const void *d_w, const int32_t *d_ids, const int8_t *d_aq,
                                        const float *d_ad, float *d_out, int blocks, int rows,
                                        int n_used, int nsub) {
    (void)nsub;
    llamd_fwd_matvec_grouped_pa(d_w, d_ids, d_aq, d_ad, d_out, blocks, rows, n_used);
}

void llamd_fwd_rms_norm_mul(const float *x, const float *w, float *out, int n, float eps) {
    if (launch_rms_norm_mul(x, w, out, 1, n, n, eps, stream())) {
        fail("rms_norm_mul: n must be in 1..8192");
        fwd_refused();
    }
}

void llamd_fwd_head_rms_norm_mul(const float *x, const float *w, float *out, int n_head, int hd,
                                 float eps) {
    if (launch_rms_norm_mul(x, w, out, n_head, hd, hd, eps, stream())) {
        fail("head_rms_norm_mul: need n_head > 0 and hd in 1..8192");
        fwd_refused();
    }
}

void llamd_fwd_rms_norm_quant(const float *x, const float *w, float *out, int8_t *qs, float *d,
                              float *inv_scratch, int n, float eps) {
    if (launch_rms_norm_quant(x, w, out, qs, d, inv_scratch, n, eps, stream())) {
        fail("rms_norm_quant: n must be a multiple of 256, at most 8192");
        fwd_refused();
    }
}

void llamd_fwd_moe_combine(const float *d, const float *weights, float *out, int n_used,
                           int n_embd) {
    checked(launch_moe_combine(d, weights, nullptr, out, n_used, n_embd, 1, stream()),
            "moe_combine (n_used 1..16)");
}

void llamd_fwd_moe_combine_add(const float *d, const float *weights, const float *residual,
                               float *out, int n_used, int n_embd) {
    checked(launch_moe_combine(d, weights, residual, out, n_used, n_embd, 1, stream()),
            "moe_combine_add (n_used 1..16)");
}

void llamd_fwd_argmax(const float *x, int n, float *scratch_v, int32_t *scratch_i, int32_t *out,
                      int nblocks) {
    // partials: one per 4096 values, at most nblocks (the caller's scratch size)
    checked(nblocks <= 0 ? -1 : launch_argmax(x, n, n, 1, scratch_v, (int *)scratch_i, out, stream(), nblocks),
            "argmax");
}

void llamd_fwd_matvec_f32(const float *w, const float *x, float *out, int k, int rows) {
    checked(launch_matvec_f32_exact(w, x, out, rows, k, 1, stream()), "matvec_f32");
}

void llamd_hip_fwd_matvec_q8_0(const void *d_w, const float *d_x, float *d_out, int rows, int k) {
    checked(launch_q8_0_mv(d_w, d_x, d_out, rows, k, stream()), "matvec_q8_0");
}

}  // extern "C"

// ---- MoE layer -------------------------------------------------------------------
namespace {


struct MoeLayer {
    int n_embd, n_ff, n_expert, n_used;
    int be, bf;  // 256-blocks per row of gate/up (n_embd) and down (n_ff)
    DevBuf router;
    void *gate = nullptr, *upw = nullptr, *downw = nullptr;
    size_t sgu = 0, sd = 0;  // expert strides
    // decode scratch
    DevBuf xq, xd, logits, ids, weights, stats;
    DevBuf g, aq, ad, dn;
    DevBuf est, slots, spec_ids;  // decode: logit estimates, hand-off words, act-row experts
    // logits [cap_seq][n_expert], ids / weights / spec_ids [cap_seq][n_used],
    // g [cap_seq][2][n_used][n_ff], est / slots [cap_seq][2][n_expert]
    // the two-launch decode kernels (moe_decode.hip) take this layer
    bool decode_fits() const { return bf <= 8 && be <= 8; }
    // prefill scratch (grown on demand)
    int cap_tok = 0, cap_seq = 1;  // prefill tokens; decode sequences (logits .. slots below)
    DevBuf p_xq, p_xd, p_grp_e, p_grp_s, p_grp_c, p_sub, p_slot, p_idx, p_g, p_u, p_aq, p_ad, p_dn;
};

// The decode kernels' arguments for this layer's scratch.
MoeDecodeLaunch decode_launch(MoeLayer *m, const float *d_x, const float *d_res, float *d_out) {
    MoeDecodeLaunch dl;
    dl.w_gate = m->gate;
    dl.w_up = m->upw;
    dl.w_down = m->downw;
    dl.gu_stride = m->sgu;
    dl.down_stride = m->sd;
    dl.router = m->router.as<float>();
    dl.x = d_x;
    dl.res = d_res;
    dl.out = d_out;
    dl.logits = m->logits.as<float>();
    dl.est = m->est.as<double>();
    dl.slots = m->slots.as<unsigned long long>();
    dl.act = m->g.as<float>();
    dl.spec_ids = m->spec_ids.as<int32_t>();
    dl.ids_out = m->ids.as<int32_t>();
    dl.w_out = m->weights.as<float>();
    dl.stats = m->stats.as<int>();
    dl.k = m->n_embd;
    dl.n_expert = m->n_expert;
    dl.n_used = m->n_used;
    dl.n_ff = m->n_ff;
    dl.polls = g_tune_moe_polls;
    return dl;
}

}  // namespace

const float *llamd::moe_router(void *h) {
    const MoeLayer *m = (const MoeLayer *)h;
    return m ? (const float *)m->router.p : nullptr;
}

int llamd::moe_router_rows(void *h) {
    const MoeLayer *m = (const MoeLayer *)h;
    return m ? m->n_expert : 0;
}

bool llamd::moe_normed_applies(void *h) {
    const MoeLayer *m = (const MoeLayer *)h;
    return m && m->decode_fits();
}

int llamd::moe_forward_normed(void *h, const float *x, const float *o, const float *w, float eps,
                              float *sum_out, float *out) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !x || !o || !w || !sum_out || !out) return fail("moe_forward_normed: null argument");
    if (!m->decode_fits()) return fail("moe_forward_normed: the layer's shapes need separate launches");
    MoeDecodeLaunch dl = decode_launch(m, sum_out, sum_out, out);
    dl.norm_a = x;
    dl.norm_b = o;
    dl.norm_w = w;
    dl.norm_eps = eps;
    dl.norm_sum = sum_out;
    return launch_moe_decode(dl, stream());
}

namespace {

// Decode scratch for nseq sequences (the stream is drained first: no queued
// kernel still reads the old buffers). The hand-off words start empty.
bool grow_decode(MoeLayer *m, int nseq) {
    if (nseq <= m->cap_seq) return true;
    if (!sync()) return false;
    const size_t n = (size_t)nseq;
    bool ok = m->logits.alloc(n * m->n_expert * 4) && m->ids.alloc(n * m->n_used * 4) &&
              m->weights.alloc(n * m->n_used * 4) && m->spec_ids.alloc(n * m->n_used * 4) &&
              m->g.alloc(n * 2 * m->n_used * m->n_ff * 4) && m->est.alloc(n * 2 * m->n_expert * 8) &&
              m->slots.alloc(n * 2 * m->n_expert * 8);
    if (ok) {
        std::vector<unsigned long long> empty(n * 2 * m->n_expert, ~0ull);
        ok = up(m->slots.p, empty.data(), empty.size() * 8) && sync();
    }
    if (!ok) {
        m->cap_seq = 0;
        return fail("moe: decode scratch for %d sequences could not be allocated", nseq) == 0;
    }
    m->cap_seq = nseq;
    return true;
}

}  // namespace

extern "C" {

void *llamd_hip_moe_create(const float *router, const void *gate, const void *upw,
                           const void *downw, int n_embd, int n_ff, int n_expert, int n_used) {
    if (!router || !gate || !upw || !downw) { fail("moe_create: null weight"); return nullptr; }
    if (n_embd <= 0 || n_ff <= 0 || n_embd % QK || n_ff % QK || n_embd > 2048) {
        fail("moe_create: n_embd and n_ff must be multiples of 256, n_embd <= 2048");
        return nullptr;
    }
    if (n_expert <= 0 || n_expert > 256 || n_used <= 0 || n_used > n_expert || n_used > 16) {
        fail("moe_create: need 0 < n_used <= n_expert <= 256, n_used <= 16");
        return nullptr;
    }
    MoeLayer *m = new MoeLayer();
    m->n_embd = n_embd; m->n_ff = n_ff; m->n_expert = n_expert; m->n_used = n_used;
    m->be = n_embd / QK; m->bf = n_ff / QK;
    bool ok = m->router.alloc((size_t)n_expert * n_embd * 4) &&
              up(m->router.p, router, (size_t)n_expert * n_embd * 4);
    m->gate = ok ? llamd_rocm_upload_q6k_experts(gate, n_expert, n_ff, m->be) : nullptr;
    m->upw = m->gate ? llamd_rocm_upload_q6k_experts(upw, n_expert, n_ff, m->be) : nullptr;
    m->downw = m->upw ? llamd_rocm_upload_q6k_experts(downw, n_expert, n_embd, m->bf) : nullptr;
    ok = ok && m->downw;
    if (ok) {
        m->sgu = llamd_hip_q6k_tiled_bytes(n_ff, m->be);
        m->sd = llamd_hip_q6k_tiled_bytes(n_embd, m->bf);
        ok = m->xq.alloc(n_embd) && m->xd.alloc(m->be * 4) &&
             m->logits.alloc(n_expert * 4) && m->ids.alloc(n_used * 4) &&
             m->weights.alloc(n_used * 4) && m->stats.alloc(16) &&
             m->g.alloc((size_t)2 * n_used * n_ff * 4) &&
             m->aq.alloc((size_t)n_used * n_ff) && m->ad.alloc((size_t)n_used * m->bf * 4) &&
             m->dn.alloc((size_t)n_used * n_embd * 4) &&
             m->est.alloc((size_t)n_expert * 16) && m->slots.alloc((size_t)n_expert * 16) &&
             m->spec_ids.alloc(n_used * 4);
        int zero[4] = {0, 0, 0, 0};
        std::vector<unsigned long long> empty((size_t)2 * n_expert, ~0ull);
        ok = ok && up(m->stats.p, zero, sizeof zero) &&
             up(m->slots.p, empty.data(), empty.size() * 8) && sync();
    }
    if (!ok) {
        llamd_hip_moe_destroy(m);
        if (!g_err[0]) fail("moe_create: allocation failed");
        return nullptr;
    }
    return m;
}

void llamd_hip_moe_destroy(void *h) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m) return;
    (void)hipStreamSynchronize(stream());
    llamd_rocm_release(m->gate);
    llamd_rocm_release(m->upw);
    llamd_rocm_release(m->downw);
    delete m;
}

int llamd_hip_moe_forward(void *h, const float *d_x, const float *d_res, float *d_out, int flags) {
    // every call is bit-exact; flags (bit 0 once asked for that) is accepted
    // and has no effect
    (void)flags;
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !d_x || !d_out) return fail("moe_forward: null argument");
    hipStream_t st = stream();
    int rc = 0;
    // 1. the reference's router logits + Q8_K of x
    RouterLaunch rl;
    rl.w = m->router.as<float>();
    rl.x = d_x;
    rl.n_expert = m->n_expert;
    rl.k = m->n_embd;
    rl.logits = m->logits.as<float>();
    rl.xq = m->xq.as<int8_t>();
    rl.xd = m->xd.as<float>();
    rl.xblocks = m->be;
    if (m->decode_fits()) {
        // router and gate/up overlapped, then down + combine (moe_decode.hip)
        MoeDecodeLaunch dl = decode_launch(m, d_x, d_res, d_out);
        rc |= launch_moe_decode(dl, st);
        return rc ? fail("moe_forward: launch failed") : 0;
    }
    // n_ff beyond the decode kernel's LDS (more than 8 blocks): one launch
    // per step of the reference's chain
    rc |= launch_router(rl, st);
    // 2. route (prologue) + gate and up of the routed experts in one
    //    launch: g holds [gate | up] x n_used x n_ff
    rc |= launch_q6k_mv_routed(m->gate, m->upw, m->sgu, m->logits.as<float>(), m->n_expert,
                               m->n_used, m->ids.as<int32_t>(), m->weights.as<float>(),
                               m->stats.as<int>(), m->xq.as<int8_t>(), m->xd.as<float>(),
                               m->g.as<float>(), m->n_ff, m->be, st);
    // 3. SwiGLU + Q8_K of the activations
    rc |= launch_swiglu_q8k(m->g.as<float>(), m->g.as<float>() + (size_t)m->n_used * m->n_ff,
                            nullptr, m->aq.as<int8_t>(), m->ad.as<float>(), nullptr,
                            m->n_used * m->bf, st);
    // 4. down projection of the routed experts + weighted combine + residual
    rc |= launch_q6k_down_combine(m->downw, m->sd, m->ids.as<int32_t>(), m->aq.as<int8_t>(),
                                  m->ad.as<float>(), m->weights.as<float>(), d_res, d_out,
                                  m->n_embd, m->bf, m->n_used, st);
    return rc ? fail("moe_forward: launch failed") : 0;
}

int llamd_hip_moe_forward_host(void *h, const float *x, const float *res, float *out, int32_t *ids,
                               float *weights, float *logits, int flags) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !x || !out) return fail("moe_forward_host: null argument");
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t nb = (size_t)m->n_embd * 4;
    DevBuf dx(nb), dr(nb), dout(nb);
    if (!dx.p || !dr.p || !dout.p) return fail("hipMalloc");
    if (!up(dx.p, x, nb)) return -1;
    if (res && !up(dr.p, res, nb)) return -1;
    if (llamd_hip_moe_forward(m, dx.as<float>(), res ? dr.as<float>() : nullptr, dout.as<float>(),
                              flags))
        return -1;
    if (!down(out, dout.p, nb)) return -1;
    if (ids && !down(ids, m->ids.p, (size_t)m->n_used * 4)) return -1;
    if (weights && !down(weights, m->weights.p, (size_t)m->n_used * 4)) return -1;
    if (logits && !down(logits, m->logits.p, (size_t)m->n_expert * 4)) return -1;
    return sync() ? 0 : -1;
}

int llamd_hip_moe_counters(void *h, int *counters, double *estimates) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !counters) return fail("moe_counters: null argument");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!down(counters, m->stats.p, 16)) return -1;
    if (estimates && !down(estimates, m->est.p, (size_t)m->n_expert * 16)) return -1;
    return sync() ? 0 : -1;
}

int llamd_hip_moe_stats(void *h, int *calls, int *exact_calls) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m) return fail("moe_stats: null handle");
    std::lock_guard<std::mutex> lk(g_mu);
    int s[4];
    if (!down(s, m->stats.p, sizeof s) || !sync()) return -1;
    if (calls) *calls = s[0];
    if (exact_calls) *exact_calls = s[1];
    // s[3] (a wait that gave up and computed the logit itself) is a timing
    // diagnostic only: the results are the same bits either way
    return 0;
}

}  // extern "C"

namespace {

// The expert-grouped FFN of n_tok tokens with routing ids / weights
// [n_tok][n_used] on the device; out = res + moe_ffn (res optional).
int moe_grouped(MoeLayer *m, const float *d_x, const int32_t *d_ids, const float *d_w,
                const float *d_res, float *d_out, int n_tok, bool fast = false) {
    const int np = n_tok * m->n_used;
    if (n_tok > m->cap_tok) {
        // grown outside any capture; the stream is drained first so no queued
        // kernel still reads the old buffers
        if (!sync()) return -1;
        const size_t NP = (size_t)np;
        const int chunks = np / CHUNK + m->n_expert;  // bound on sum of ceil(count/16)
        bool ok = m->p_xq.alloc((size_t)chunks * m->be * CHUNK_BLOCK) &&
                  m->p_xd.alloc((size_t)chunks * m->be * CHUNK * 4) &&
                  m->p_grp_e.alloc(m->n_expert * 4) && m->p_grp_s.alloc(m->n_expert * 4) &&
                  m->p_grp_c.alloc(m->n_expert * 4) && m->p_sub.alloc((group_items_offset(m->n_expert) + 2 * (size_t)chunks * 8) * 4) &&
                  m->p_slot.alloc(NP * 4) && m->p_idx.alloc(NP * 4) &&
                  m->p_g.alloc(NP * m->n_ff * 4) && m->p_u.alloc(NP * m->n_ff * 4) &&
                  m->p_aq.alloc((size_t)chunks * m->bf * CHUNK_BLOCK) &&
                  m->p_ad.alloc((size_t)chunks * m->bf * CHUNK * 4) &&
                  m->p_dn.alloc(NP * m->n_embd * 4);
        if (!ok) { m->cap_tok = 0; return fail("moe_prefill: allocation failed"); }
        m->cap_tok = n_tok;
    }
    hipStream_t st = stream();
    const int max_chunks = np / CHUNK + m->n_expert;
    int rc = 0;
    rc |= launch_moe_group(d_ids, np, m->n_used, m->n_expert, m->p_grp_e.as<int32_t>(),
                           m->p_grp_s.as<int32_t>(), m->p_grp_c.as<int32_t>(),
                           m->p_sub.as<int32_t>(), m->p_slot.as<int32_t>(), m->p_idx.as<int32_t>(),
                           st, max_chunks);
    // Q8_K of every token, written to the chunk slot of each of its n_used pairs
    rc |= launch_q8k_quantize_chunks(d_x, n_tok, m->be, m->p_slot.as<int32_t>(), m->n_used,
                                     m->p_xq.as<int8_t>(), m->p_xd.as<float>(), st);
    // gate / up: output row = the pair index
    // gate and up in one launch (same shapes, same activations)
    rc |= launch_q6k_mv_batched(m->gate, m->sgu, m->p_grp_e.as<int32_t>(), m->p_grp_s.as<int32_t>(),
                                m->p_grp_c.as<int32_t>(), m->p_sub.as<int32_t>(),
                                m->p_idx.as<int32_t>(), m->p_xq.as<int8_t>(), m->p_xd.as<float>(),
                                m->p_g.as<float>(), m->n_ff, m->n_ff, m->be, m->n_expert, max_chunks, st,
                                nullptr, nullptr, true, m->upw, m->p_u.as<float>(), fast);
    // SwiGLU + Q8_K per pair, into the pair's chunk slot
    rc |= launch_swiglu_q8k_chunks(m->p_g.as<float>(), m->p_u.as<float>(), np, m->bf,
                                   m->p_slot.as<int32_t>(), m->p_aq.as<int8_t>(),
                                   m->p_ad.as<float>(), st);
    // down: output row = the pair index
    rc |= launch_q6k_mv_batched(m->downw, m->sd, m->p_grp_e.as<int32_t>(), m->p_grp_s.as<int32_t>(),
                                m->p_grp_c.as<int32_t>(), m->p_sub.as<int32_t>(),
                                m->p_idx.as<int32_t>(), m->p_aq.as<int8_t>(), m->p_ad.as<float>(),
                                m->p_dn.as<float>(), m->n_embd, m->n_embd, m->bf, m->n_expert,
                                max_chunks, st, nullptr, nullptr, true, nullptr, nullptr, fast);
    rc |= launch_moe_combine(m->p_dn.as<float>(), d_w, d_res, d_out, m->n_used, m->n_embd, n_tok, st,
                             m->p_slot.as<int32_t>());
    return rc ? fail("moe_prefill: launch failed") : 0;
}

}  // namespace

extern "C" {

int llamd_hip_moe_prefill(void *h, const float *d_x, const int32_t *d_ids, const float *d_w,
                          float *d_out, int n_tok) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !d_x || !d_ids || !d_w || !d_out || n_tok <= 0) return fail("moe_prefill: bad arguments");
    return moe_grouped(m, d_x, d_ids, d_w, nullptr, d_out, n_tok);
}

int llamd_hip_moe_prefill_ex(void *h, const float *d_x, const int32_t *d_ids, const float *d_w,
                             float *d_out, int n_tok, int flags) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !d_x || !d_ids || !d_w || !d_out || n_tok <= 0 || (flags & ~LLAMD_HIP_REDUCTION))
        return fail("moe_prefill_ex: bad arguments");
    return moe_grouped(m, d_x, d_ids, d_w, nullptr, d_out, n_tok, (flags & LLAMD_HIP_REDUCTION) != 0);
}

int llamd_hip_moe_forward_batch(void *h, const float *d_x, const float *d_res, float *d_out,
                                int nseq) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !d_x || !d_out || nseq <= 0) return fail("moe_forward_batch: bad arguments");
    if (!grow_decode(m, nseq)) return -1;
    hipStream_t st = stream();
    if (nseq <= g_tune_batch_decode_max && m->decode_fits()) {
        // the decode kernels over the batch: per sequence, router fold beside
        // gate/up, then down + ordered combine (two launches for the batch)
        MoeDecodeLaunch dl = decode_launch(m, d_x, d_res, d_out);
        dl.nseq = nseq;
        return launch_moe_decode(dl, st) ? fail("moe_forward_batch: launch failed") : 0;
    }
    // 1. the reference's router logits for every (sequence, expert), all folds at once
    RouterLaunch rl;
    rl.w = m->router.as<float>();
    rl.x = d_x;
    rl.n_expert = m->n_expert;
    rl.k = m->n_embd;
    rl.logits = m->logits.as<float>();
    rl.xq = nullptr;
    rl.xd = nullptr;
    rl.xblocks = 0;
    rl.nseq = nseq;
    int rc = launch_router(rl, st);
    // 2. softmax / top-k / renormalise per sequence
    rc |= launch_route_logits(m->logits.as<float>(), m->n_expert, m->n_used, m->ids.as<int32_t>(),
                              m->weights.as<float>(), st, nseq);
    if (rc) return fail("moe_forward_batch: launch failed");
    // 3. the experts grouped across the sequences (an expert's weights read
    //    once per 16 tokens routed to it), combine + residual
    return moe_grouped(m, d_x, m->ids.as<int32_t>(), m->weights.as<float>(), d_res, d_out, nseq);
}

int llamd_hip_moe_forward_batch_host(void *h, const float *x, const float *res, float *out,
                                     int32_t *ids, float *weights, float *logits, int nseq) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !x || !out || nseq <= 0) return fail("moe_forward_batch_host: bad arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t nb = (size_t)nseq * m->n_embd * 4;
    DevBuf dx(nb), dr(nb), dout(nb);
    if (!dx.p || !dr.p || !dout.p) return fail("hipMalloc");
    if (!up(dx.p, x, nb)) return -1;
    if (res && !up(dr.p, res, nb)) return -1;
    if (llamd_hip_moe_forward_batch(m, dx.as<float>(), res ? dr.as<float>() : nullptr,
                                    dout.as<float>(), nseq))
        return -1;
    if (!down(out, dout.p, nb)) return -1;
    if (ids && !down(ids, m->ids.p, (size_t)nseq * m->n_used * 4)) return -1;
    if (weights && !down(weights, m->weights.p, (size_t)nseq * m->n_used * 4)) return -1;
    if (logits && !down(logits, m->logits.p, (size_t)nseq * m->n_expert * 4)) return -1;
    return sync() ? 0 : -1;
}

int llamd_hip_moe_prefill_host(void *h, const float *x, const int32_t *ids, const float *w,
                               float *out, int n_tok) {
    return llamd_hip_moe_prefill_host_ex(h, x, ids, w, out, n_tok, 0);
}

int llamd_hip_moe_prefill_host_ex(void *h, const float *x, const int32_t *ids, const float *w,
                                  float *out, int n_tok, int flags) {
    MoeLayer *m = (MoeLayer *)h;
    if (!m || !x || !ids || !w || !out || n_tok <= 0 || (flags & ~LLAMD_HIP_REDUCTION))
        return fail("moe_prefill_host: bad arguments");
    const int np = n_tok * m->n_used;
    for (int i = 0; i < np; ++i)
        if (ids[i] < 0 || ids[i] >= m->n_expert) return fail("moe_prefill_host: bad expert id %d", ids[i]);
    std::lock_guard<std::mutex> lk(g_mu);
    const size_t nx = (size_t)n_tok * m->n_embd * 4;
    DevBuf dx(nx), di((size_t)np * 4), dw((size_t)np * 4), dout(nx);
    if (!dx.p || !di.p || !dw.p || !dout.p) return fail("hipMalloc");
    if (!up(dx.p, x, nx) || !up(di.p, ids, (size_t)np * 4) || !up(dw.p, w, (size_t)np * 4)) return -1;
    if (llamd_hip_moe_prefill_ex(m, dx.as<float>(), di.as<int32_t>(), dw.as<float>(), dout.as<float>(),
                                 n_tok, flags))
        return -1;
    if (!down(out, dout.p, nx) || !sync()) return -1;
    return 0;
}

}  // extern "C"

// ---- LM head ---------------------------------------------------------------------
namespace {
}  // namespace

// The LM-head call's launches on the library stream: Q8_K of x, the Q6_K
// matvec whose epilogue leaves one arg-max candidate per 16-row tile, and
// the reduction of the candidates.
int llamd::lmhead_enqueue(const void *w, int rows, int blocks, const float *d_x, int nseq,
                          float *d_logits, int32_t *d_ids, const LmHeadScratch &sc) {
    hipStream_t st = stream();
    int rc = 0;
    const int tiles = (rows + 15) / 16;
    if (nseq == 1) {
        rc |= launch_q8k_quantize(d_x, sc.xq, sc.xd, nullptr, blocks, st);
        rc |= launch_q6k_mv_b1(w, 0, nullptr, sc.xq, sc.xd, d_logits, rows, blocks, 1, 0, st,
                               nullptr, sc.pv, sc.pi);
    } else if (sc.mt) {
        // REDUCTION-tolerance logits; the arg-max is certified and exact
        rc |= launch_q8k_quantize_chunks(d_x, nseq, blocks, nullptr, 1, sc.cq, sc.cd, st, sc.xq, sc.xd);
        rc |= launch_q6k_mv_batched(w, 0, nullptr, nullptr, nullptr, nullptr, nullptr, sc.cq, sc.cd,
                                    d_logits, rows, rows, blocks, nseq, (nseq + CHUNK - 1) / CHUNK,
                                    st, sc.pv, sc.pi, false, nullptr, nullptr, true);
        rc |= launch_lmhead_certify(w, rows, blocks, nseq, sc.xq, sc.xd, sc.pv, sc.pi, sc.mt,
                                    d_logits, d_ids, st);
        return rc;
    } else {
        rc |= launch_q8k_quantize_chunks(d_x, nseq, blocks, nullptr, 1, sc.cq, sc.cd, st);
        rc |= launch_q6k_mv_batched(w, 0, nullptr, nullptr, nullptr, nullptr, nullptr, sc.cq, sc.cd,
                                    d_logits, rows, rows, blocks, nseq, (nseq + CHUNK - 1) / CHUNK,
                                    st, sc.pv, sc.pi);
    }
    rc |= launch_argmax_final(d_logits, rows, nseq, sc.pv, sc.pi, tiles, d_ids, st);
    return rc;
}

size_t llamd::lmhead_chunk_q_bytes(int nseq, int blocks) { return chunk_q_bytes(nseq, blocks); }
size_t llamd::lmhead_chunk_d_bytes(int nseq, int blocks) { return chunk_d_bytes(nseq, blocks); }

int llamd::q6k_handle_shape(const void *p, int *rows, int *blocks, int *n_expert) {
    WInfo wi;
    if (!lookup(p, KIND_Q6K, &wi)) return -1;
    *rows = wi.rows;
    *blocks = wi.blocks;
    *n_expert = wi.n_expert;
    return 0;
}

hipStream_t llamd::lib_stream() { return stream(); }

namespace {
struct LmHead {
    const void *w;
    int rows, blocks, cap;
    DevBuf xq, xd, cq, cd, pv, pi;  // cq, cd: chunked activations for nseq > 1
    DevBuf mt;                      // per-tile weight bound (LLAMD_HIP_REDUCTION)
};
}  // namespace

int llamd::lmhead_forward_q8k(void *h, const int8_t *xq, const float *xd, float *d_logits,
                              int32_t *d_ids) {
    LmHead *l = (LmHead *)h;
    if (!l || !xq || !xd || !d_logits || !d_ids) return fail("lmhead_forward_q8k: bad arguments");
    hipStream_t st = stream();
    int rc = launch_q6k_mv_b1(l->w, 0, nullptr, xq, xd, d_logits, l->rows, l->blocks, 1, 0, st,
                              nullptr, l->pv.as<float>(), l->pi.as<int>());
    rc |= launch_argmax_final(d_logits, l->rows, 1, l->pv.as<float>(), l->pi.as<int>(),
                              (l->rows + 15) / 16, d_ids, st);
    return rc ? fail("lmhead_forward_q8k: launch failed") : 0;
}

extern "C" {

void *llamd_hip_lmhead_create(const void *d_w, int rows, int blocks, int max_seq) {
    WInfo wi;
    if (lookup(d_w, KIND_Q6K, &wi) && (wi.n_expert != 1 || wi.rows != rows || wi.blocks != blocks)) {
        fail("lmhead_create: weight handle does not match rows=%d blocks=%d", rows, blocks);
        return nullptr;
    }
    Q6kView v;
    if (resolve_q6k(d_w, nullptr, rows, blocks, false, &v)) return nullptr;
    if (max_seq <= 0) { fail("lmhead_create: max_seq must be positive"); return nullptr; }
    LmHead *l = new LmHead();
    l->w = v.tiled; l->rows = rows; l->blocks = blocks; l->cap = max_seq;

    // per-tile arg-max candidates written by the matvec epilogue
    const int parts = (rows + 15) / 16;
    const size_t nq = (size_t)max_seq * blocks * QK;
    if (!l->xq.alloc(nq) || !l->xd.alloc((size_t)max_seq * blocks * 4) ||
        !l->cq.alloc(chunk_q_bytes(max_seq, blocks)) || !l->cd.alloc(chunk_d_bytes(max_seq, blocks)) ||
        !l->pv.alloc((size_t)parts * max_seq * 4) || !l->pi.alloc((size_t)parts * max_seq * 4) ||
        !l->mt.alloc((size_t)parts * 4)) {
        delete l;
        fail("lmhead_create: allocation failed");
        return nullptr;
    }
    // the weights' per-tile bound, once (read by the certified arg-max)
    if (launch_q6k_tile_bound(l->w, rows, blocks, l->mt.as<float>(), stream()) || !sync()) {
        delete l;
        fail("lmhead_create: tile bound failed");
        return nullptr;
    }
    return l;
}

void llamd_hip_lmhead_destroy(void *h) {
    if (!h) return;
    (void)hipStreamSynchronize(stream());
    delete (LmHead *)h;
}

int llamd_hip_lmhead_forward(void *h, const float *d_x, int nseq, float *d_logits, int32_t *d_ids) {
    return llamd_hip_lmhead_forward_ex(h, d_x, nseq, d_logits, d_ids, 0);
}

int llamd_hip_lmhead_forward_ex(void *h, const float *d_x, int nseq, float *d_logits, int32_t *d_ids,
                                int flags) {
    LmHead *l = (LmHead *)h;
    if (!l || !d_x || !d_logits || !d_ids || nseq <= 0 || nseq > l->cap || (flags & ~LLAMD_HIP_REDUCTION))
        return fail("lmhead_forward: bad arguments");
    LmHeadScratch sc{l->xq.as<int8_t>(), l->xd.as<float>(), l->cq.as<int8_t>(), l->cd.as<float>(),
                     l->pv.as<float>(), l->pi.as<int>()};
    if ((flags & LLAMD_HIP_REDUCTION) && nseq > 1) sc.mt = l->mt.as<float>();
    return lmhead_enqueue(l->w, l->rows, l->blocks, d_x, nseq, d_logits, d_ids, sc)
               ? fail("lmhead_forward: launch failed") : 0;
}

// ---- timing ----------------------------------------------------------------------
void *llamd_hip_event_create(void) {
    hipEvent_t e = nullptr;
    if (!hip_ok(hipEventCreate(&e), "hipEventCreate")) return nullptr;
    return (void *)e;
}
void llamd_hip_event_destroy(void *ev) {
    if (ev) (void)hipEventDestroy((hipEvent_t)ev);
}
int llamd_hip_event_record(void *ev) {
    return hip_ok(hipEventRecord((hipEvent_t)ev, stream()), "hipEventRecord") ? 0 : -1;
}
float llamd_hip_event_elapsed_ms(void *a, void *b) {
    float ms = -1.f;
    if (hipEventSynchronize((hipEvent_t)b) != hipSuccess) return -1.f;
    if (hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b) != hipSuccess) return -1.f;
    return ms;
}

static int bench_common(const void *d_w, const int32_t *eid, const int8_t *aq, const float *ad,
                        int blocks, int rows, int n_used, int iters, float *ms_out) {
    if (iters <= 0 || !ms_out || !aq || !ad) return fail("bench: bad arguments");
    size_t stride = 0;
    int ne = 1;
    if (eid) {
        if (expert_view(d_w, rows, blocks, &stride, &ne, &d_w)) return -1;
        for (int i = 0; i < n_used; ++i)
            if (eid[i] < 0 || eid[i] >= ne) return fail("bench: bad expert id");
    } else {
        Q6kView v;
        if (resolve_q6k(d_w, nullptr, rows, blocks, false, &v)) return -1;
        d_w = v.tiled;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    DevBuf q((size_t)blocks * QK), d((size_t)blocks * 4), y((size_t)rows * n_used * 4),
        ids((size_t)n_used * 4);
    if (!q.p || !d.p || !y.p || !ids.p) return fail("hipMalloc");
    if (!up(q.p, aq, (size_t)blocks * QK) || !up(d.p, ad, (size_t)blocks * 4)) return -1;
    if (eid && !up(ids.p, eid, (size_t)n_used * 4)) return -1;
    hipStream_t st = stream();
    auto launch = [&]() {
        return launch_q6k_mv_b1(d_w, stride, eid ? ids.as<int32_t>() : nullptr, q.as<int8_t>(),
                                d.as<float>(), y.as<float>(), rows, blocks, n_used, 0, st);
    };
    if (launch() || !sync()) return fail("bench: warm launch failed");
    hipEvent_t t0, t1;
    if (hipEventCreate(&t0) != hipSuccess) return fail("hipEventCreate");
    if (hipEventCreate(&t1) != hipSuccess) { (void)hipEventDestroy(t0); return fail("hipEventCreate"); }
    int rc = -1;
    if (hipEventRecord(t0, st) == hipSuccess) {
        int bad = 0;
        for (int i = 0; i < iters; ++i) bad |= launch();
        if (!bad && hipEventRecord(t1, st) == hipSuccess && hipEventSynchronize(t1) == hipSuccess &&
            hipEventElapsedTime(ms_out, t0, t1) == hipSuccess)
            rc = 0;
    }
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    return rc ? fail("bench: timing failed") : 0;
}

int llamd_hip_read_many(const void *const *d_src, size_t bytes, int grid, int n) {
    if (n < 0 || grid < 1 || bytes % 16 || (n && bytes && !d_src))
        return fail("read_many: bad arguments (bytes a multiple of 16, grid >= 1)");
    for (int i = 0; i < n; ++i)
        if (launch_read_calibration(bytes ? d_src[i] : nullptr, bytes, grid, stream()))
            return fail("read_many: launch %d failed", i);
    return 0;
}

int llamd_hip_copy_calibration(void *d_dst, const void *d_src, size_t bytes) {
    if (!d_dst || !d_src || bytes % 16) return fail("copy_calibration: bytes must be a multiple of 16");
    return launch_copy_calibration(d_dst, d_src, bytes, stream()) ? fail("copy_calibration: launch") : 0;
}

int llamd_rocm_matvec_bench(const void *d_w, const int8_t *aq, const float *ad, int blocks,
                            int rows, int iters, float *ms_out) {
    return bench_common(d_w, nullptr, aq, ad, blocks, rows, 1, iters, ms_out);
}

int llamd_rocm_matvec_grouped_bench(const void *d_w, const int32_t *eid, const int8_t *aq,
                                    const float *ad, int blocks, int rows, int n_used, int iters,
                                    float *ms_out) {
    if (n_used <= 0 || !eid) return fail("grouped bench: no experts");
    return bench_common(d_w, eid, aq, ad, blocks, rows, n_used, iters, ms_out);
}

}  // extern "C"
