// compat_abi.cpp -- the rest of the C ABI that crates/llamd-rocm binds
// (src/forward.rs:269-616, src/batch.rs:43-180, src/udot.rs:15-150), so that
// the reference's Rust crate links against this library unchanged, plus
// row-wise f32 entry points for the llamd-tensor Backend trait
// (crates/llamd-tensor/src/lib.rs:148-174).
//
// Q6_K weights. The reference keeps Q6_K tensors in its own device layouts:
// ggml's 210-byte blocks (DevBuf::from_bytes, used by llamd_fwd_matvec* and
// llamd_b_*) and the planar repack (PlanarWeights, used by llamd_fwd_planar_*
// and llamd_u_*). This file keeps a tiled copy of each such tensor
// (compat.hip q6k_retile) in the layout the MFMA kernels read, made the first
// time an entry point is handed the tensor and re-made whenever the library
// itself writes the bytes (llamd_fwd_upload, llamd_fwd_memset); freeing the
// allocation (llamd_fwd_free, llamd_rocm_release) frees the copy. The source
// must lie in memory from llamd_fwd_alloc or llamd_rocm_upload, whose extents
// this file records, so the copy never reads past an allocation. The copy
// doubles the tensor's footprint (24 GB more for a Qwen3-30B-A3B-sized
// model, on a 288 GB device). Under graph capture the first use allocates the
// copy and fills it on a side stream, which the capture mode (relaxed) allows.
//
// Activations. llamd_b_* and llamd_fwd_* take the reference's natural Q8_K
// arrays; llamd_u_* take them biased to unsigned (qb = q ^ 0x80, with per-16
// sums sb, which this backend does not need). Batches of more than one
// sequence are regrouped into the token-chunked operand layout of the
// batched MFMA kernel in a library-owned scratch buffer. Every result is the
// bit-exact signed computation of dot_q6k_q8k (crates/llamd-quant/src/
// dot.rs:138-196), which lies within the REDUCTION tolerance the reference
// allows its own udot path.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/llamd_hip.h"
#include "errors.hpp"
#include "launch.hpp"

using namespace llamd;

namespace {

constexpr int QK = 256;
constexpr int CHUNK = 16;
// Positions a RoPE table covers when the caller gives no bound (the meta
// entry points read the position on the device).
constexpr int ROPE_DEFAULT_ROWS = 32768;

// Serialises the calls that stage activations in the shared scratch, so two
// threads' staging and launches cannot interleave on the one stream.
std::mutex g_smu;
std::mutex g_cmu;  // guards everything below
std::map<uintptr_t, size_t> g_alloc;  // llamd_fwd_alloc / llamd_rocm_upload extents

struct Shadow {
    uintptr_t key;
    bool planar;
    size_t off[4];
    int blocks, rows;
    Q6kSource src;
    void *tiled;
    uintptr_t lo, hi;  // the source bytes it was made from
};
std::vector<Shadow> g_shadow;

struct RopeTab {
    int hd;
    uint32_t base_bits;
    int rows;
    float2 *d;  // [rows][hd / 2], then den [hd / 2] floats
};
std::vector<RopeTab> g_rope;
// Superseded scratch buffers a captured graph may still read, kept until the
// process ends. Scratch only grows by at least doubling, so together they
// never exceed the live scratch's size.
std::vector<void *> g_retired;

void *g_scr = nullptr;
size_t g_scr_cap = 0;
int g_u_tile = 1;

hipStream_t g_side = nullptr;

hipStream_t S() { return lib_stream(); }

hipStream_t side() {
    if (!g_side && hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking) != hipSuccess)
        g_side = nullptr;
    return g_side;
}

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return false;
    return cs == hipStreamCaptureStatusActive;
}

bool alloc_range(uintptr_t p, uintptr_t *a0, uintptr_t *a1) {
    auto it = g_alloc.upper_bound(p);
    if (it == g_alloc.begin()) return false;
    --it;
    if (p >= it->first + it->second) return false;
    *a0 = it->first;
    *a1 = it->first + it->second;
    return true;
}

// Library scratch of at least `bytes` (stream-ordered reuse; a smaller
// buffer it replaces stays allocated for graphs that captured it).
void *scratch(size_t bytes) {
    std::lock_guard<std::mutex> lk(g_cmu);
    if (bytes <= g_scr_cap) return g_scr;
    const size_t cap = std::max<size_t>({bytes, 2 * g_scr_cap, (size_t)4 << 20});
    void *p = nullptr;
    if (hipMalloc(&p, cap) != hipSuccess) {
        set_error("scratch: hipMalloc of %zu bytes", cap);
        return nullptr;
    }
    if (g_scr) g_retired.push_back(g_scr);
    g_scr = p;
    g_scr_cap = cap;
    return p;
}

// cos / sin of theta = pos / powf(base, 2i / hd) for pos in [0, rows) and
// i < hd / 2, with the host libm -- the calls the reference CPU path makes
// (crates/llamd-cpu/src/lib.rs:183-205, freq_scale 1) -- followed by the
// denominators powf(base, 2i / hd), with which head_norm_rope rotates the
// positions past the table on the device. One table of ROPE_DEFAULT_ROWS
// rows per (head_dim, base), made once: no position rebuilds it.
const float2 *rope_table(int hd, float base, int *rows_out, const float **den_out) {
    std::lock_guard<std::mutex> lk(g_cmu);
    uint32_t bits;
    memcpy(&bits, &base, 4);
    const int half = hd / 2;
    for (auto &r : g_rope)
        if (r.hd == hd && r.base_bits == bits) {
            *rows_out = r.rows;
            *den_out = (const float *)(r.d + (size_t)r.rows * half);
            return r.d;
        }
    const int rows = ROPE_DEFAULT_ROWS;
    std::vector<float> den(half);
    for (int i = 0; i < half; ++i) den[i] = powf(base, 2.0f * (float)i / (float)hd);
    std::vector<float2> cs((size_t)rows * half);
    for (int pos = 0; pos < rows; ++pos) {
        const float pf = (float)pos * 1.0f;
        for (int i = 0; i < half; ++i) {
            const float theta = pf / den[i];
            cs[(size_t)pos * half + i] = make_float2(cosf(theta), sinf(theta));
        }
    }
    float2 *d = nullptr;
    hipStream_t sd = side();
    const size_t tab_bytes = cs.size() * sizeof(float2);
    if (!sd || hipMalloc(&d, tab_bytes + half * sizeof(float)) != hipSuccess ||
        hipMemcpyAsync(d, cs.data(), tab_bytes, hipMemcpyHostToDevice, sd) != hipSuccess ||
        hipMemcpyAsync((char *)d + tab_bytes, den.data(), half * sizeof(float), hipMemcpyHostToDevice,
                       sd) != hipSuccess ||
        hipStreamSynchronize(sd) != hipSuccess) {
        set_error("rope table: device copy failed");
        return nullptr;
    }
    g_rope.push_back(RopeTab{hd, bits, rows, d});
    *rows_out = rows;
    *den_out = (const float *)((char *)d + tab_bytes);
    return d;
}

#define REFUSE(...)                 \
    do {                            \
        set_error(__VA_ARGS__);     \
        fwd_refused();              \
        return;                     \
    } while (0)

#define REFUSE_IF(cond, ...)        \
    do {                            \
        if (cond) REFUSE(__VA_ARGS__); \
    } while (0)

// Q8_K operands of n_act tokens for the Q6_K kernels: natural signed arrays
// (b1 kernels) or the token-chunked layout (batched kernel, n_act > 1).
struct Acts {
    const int8_t *q = nullptr;
    const float *d = nullptr;
    int8_t *cq = nullptr;
    float *cd = nullptr;
};

size_t chunk_q_bytes(int n, int blocks) { return (size_t)((n + CHUNK - 1) / CHUNK) * blocks * 4096; }
size_t chunk_d_bytes(int n, int blocks) { return (size_t)((n + CHUNK - 1) / CHUNK) * blocks * CHUNK * 4; }

// natural form: q as given (signed) or unbiased into scratch
int natural(const void *q, const float *d, bool biased, int n_act, int blocks, Acts *a) {
    a->d = d;
    if (!biased) {
        a->q = (const int8_t *)q;
        return 0;
    }
    int8_t *s = (int8_t *)scratch((size_t)n_act * blocks * QK);
    if (!s) return -1;
    if (launch_act_unbias(q, true, n_act, blocks, s, S())) return set_error("unbias: launch");
    a->q = s;
    return 0;
}

int chunked(const void *q, const float *d, bool biased, int n_act, int blocks, Acts *a) {
    const size_t nq = chunk_q_bytes(n_act, blocks);
    uint8_t *s = (uint8_t *)scratch(nq + chunk_d_bytes(n_act, blocks));
    if (!s) return -1;
    a->cq = (int8_t *)s;
    a->cd = (float *)(s + nq);
    if (launch_act_to_chunks(q, d, biased, n_act, blocks, a->cq, a->cd, S()))
        return set_error("chunk: launch");
    return 0;
}

// out [nseq][rows] = W . act_s for every sequence s
int matvec_n(const Q6kView &v, const Acts &a, float *out, int rows, int blocks, int nseq) {
    if (nseq == 1)
        return launch_q6k_mv_b1(v.tiled, 0, nullptr, a.q, a.d, out, rows, blocks, 1, 0, S());
    return launch_q6k_mv_batched(v.tiled, 0, nullptr, nullptr, nullptr, nullptr, nullptr, a.cq, a.cd,
                                 out, rows, rows, blocks, nseq, (nseq + CHUNK - 1) / CHUNK, S());
}

int prep(const void *q, const float *d, bool biased, int nseq, int blocks, Acts *a) {
    return nseq == 1 ? natural(q, d, biased, 1, blocks, a) : chunked(q, d, biased, nseq, blocks, a);
}

void matvec_entry(const void *w, const size_t *off, const void *q, const float *d, bool biased,
                  float *out, int blocks, int rows, int nseq) {
    std::lock_guard<std::mutex> lk(g_smu);
    REFUSE_IF(!q || !d || !out || nseq <= 0, "matvec: null operand or nseq %d", nseq);
    Q6kView v;
    Acts a;
    if (resolve_q6k(w, off, rows, blocks, false, &v) || prep(q, d, biased, nseq, blocks, &a))
        return fwd_refused();
    if (matvec_n(v, a, out, rows, blocks, nseq)) REFUSE("matvec: launch");
}

void x3_entry(const void *const w[3], const size_t *const off[3], const void *q, const float *d,
              bool biased, float *const o[3], int blocks, const int rows[3], int nseq) {
    std::lock_guard<std::mutex> lk(g_smu);
    REFUSE_IF(!q || !d || nseq <= 0, "matvec_x3: null operand or nseq %d", nseq);
    const void *t[3];
    for (int i = 0; i < 3; ++i) {
        Q6kView v;
        if (resolve_q6k(w[i], off[i], rows[i], blocks, false, &v)) return fwd_refused();
        t[i] = v.tiled;
    }
    Acts a;
    if (prep(q, d, biased, nseq, blocks, &a)) return fwd_refused();
    if (nseq == 1) {
        if (launch_q6k_mv_x3(t, o, rows, 3, a.q, a.d, blocks, S())) REFUSE("matvec_x3: launch");
        return;
    }
    if (launch_q6k_mv_batched_x3(t, o, rows, 3, a.cq, a.cd, blocks, nseq, S()))
        REFUSE("matvec_x3: launch");
}

// gate and up of nseq sequences' own experts: slot s * n_used + k reads
// activation s; oa, ob [nseq][n_used][rows]
void grouped_x2_entry(const void *wa, const size_t *fa, const void *wb, const size_t *fb,
                      const int32_t *ids, const void *q, const float *d, bool biased, float *oa,
                      float *ob, int blocks, int rows, int n_used, int nseq) {
    std::lock_guard<std::mutex> lk(g_smu);
    REFUSE_IF(!ids || !q || !d || n_used <= 0 || nseq <= 0, "grouped_x2: bad arguments");
    Q6kView va, vb;
    if (resolve_q6k(wa, fa, rows, blocks, true, &va) || resolve_q6k(wb, fb, rows, blocks, true, &vb))
        return fwd_refused();
    REFUSE_IF(va.expert_stride != vb.expert_stride, "grouped_x2: the two expert tensors differ");
    Acts a;
    if (natural(q, d, biased, nseq, blocks, &a)) return fwd_refused();
    if (launch_q6k_mv_grouped_x2(va.tiled, vb.tiled, va.expert_stride, ids, a.q, a.d, oa, ob, rows,
                                 blocks, n_used * nseq, S(), n_used))
        REFUSE("grouped_x2: launch");
}

// down: slot s * n_used + k reads activation s * n_used + k; out [nseq][n_used][rows]
void grouped_pa_entry(const void *w, const size_t *off, const int32_t *ids, const void *q,
                      const float *d, bool biased, float *out, int blocks, int rows, int n_used,
                      int nseq) {
    std::lock_guard<std::mutex> lk(g_smu);
    REFUSE_IF(!ids || !q || !d || n_used <= 0 || nseq <= 0, "grouped_pa: bad arguments");
    Q6kView v;
    if (resolve_q6k(w, off, rows, blocks, true, &v)) return fwd_refused();
    Acts a;
    if (natural(q, d, biased, nseq * n_used, blocks, &a)) return fwd_refused();
    if (launch_q6k_mv_b1(v.tiled, v.expert_stride, ids, a.q, a.d, out, rows, blocks, n_used * nseq,
                         1, S()))
        REFUSE("grouped_pa: launch");
}

void grouped_entry(const void *w, const size_t *off, const int32_t *ids, const int8_t *q,
                   const float *d, float *out, int blocks, int rows, int n_used) {
    REFUSE_IF(!ids || !q || !d || n_used <= 0, "grouped: bad arguments");
    Q6kView v;
    if (resolve_q6k(w, off, rows, blocks, true, &v)) return fwd_refused();
    if (launch_q6k_mv_b1(v.tiled, v.expert_stride, ids, q, d, out, rows, blocks, n_used, 0, S()))
        REFUSE("grouped: launch");
}

struct DevTmp {
    void *p = nullptr;
    explicit DevTmp(size_t n) {
        if (hipMalloc(&p, n ? n : 16) != hipSuccess) p = nullptr;
    }
    ~DevTmp() {
        if (p) (void)hipFree(p);
    }
    DevTmp(const DevTmp &) = delete;
    DevTmp &operator=(const DevTmp &) = delete;
};

int h2d(void *dst, const void *src, size_t n) {
    return hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, S()) == hipSuccess
               ? 0 : set_error("upload of %zu bytes failed", n);
}
int d2h(void *dst, const void *src, size_t n) {
    return hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, S()) == hipSuccess
               ? 0 : set_error("download of %zu bytes failed", n);
}
int sync_check(const char *what) {
    if (hipStreamSynchronize(S()) != hipSuccess) return set_error("%s: synchronize failed", what);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error("%s: %s", what, hipGetErrorString(e));
}

// Milliseconds for `iters` launches of `launch` (after one warm launch), with
// events on the library stream, like the reference's *_bench entry points.
template <class F>
int time_launches(F launch, int iters, float *ms_out, const char *what) {
    if (iters <= 0 || !ms_out) return set_error("%s: bad iteration count", what);
    launch();
    if (sync_check(what)) return -1;
    hipEvent_t t0, t1;
    if (hipEventCreate(&t0) != hipSuccess) return set_error("hipEventCreate");
    if (hipEventCreate(&t1) != hipSuccess) {
        (void)hipEventDestroy(t0);
        return set_error("hipEventCreate");
    }
    int rc = -1;
    if (hipEventRecord(t0, S()) == hipSuccess) {
        for (int i = 0; i < iters; ++i) launch();
        if (hipEventRecord(t1, S()) == hipSuccess && hipEventSynchronize(t1) == hipSuccess &&
            hipEventElapsedTime(ms_out, t0, t1) == hipSuccess)
            rc = 0;
    }
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (rc || sync_check(what)) return set_error("%s: timing failed", what);
    return 0;
}

// Host-in, host-out Q6_K matvec over nseq signed activations.
int host_matvec(const void *w, const size_t *off, const int8_t *qs, const float *ad, float *out,
                int blocks, int rows, int nseq) {
    std::lock_guard<std::mutex> lk(g_smu);
    if (!qs || !ad || !out || nseq <= 0) return set_error("matvec: bad arguments");
    Q6kView v;
    if (resolve_q6k(w, off, rows, blocks, false, &v)) return -1;
    DevTmp q((size_t)nseq * blocks * QK), d((size_t)nseq * blocks * 4), y((size_t)nseq * rows * 4);
    if (!q.p || !d.p || !y.p) return set_error("hipMalloc");
    Acts a;
    if (h2d(q.p, qs, (size_t)nseq * blocks * QK) || h2d(d.p, ad, (size_t)nseq * blocks * 4) ||
        prep(q.p, (const float *)d.p, false, nseq, blocks, &a) ||
        matvec_n(v, a, (float *)y.p, rows, blocks, nseq) ||
        d2h(out, y.p, (size_t)nseq * rows * 4))
        return -1;
    return sync_check("matvec");
}

int bench_matvec(const void *w, const size_t *off, const int8_t *qs, const float *ad, int blocks,
                 int rows, int nseq, int iters, float *ms_out) {
    std::lock_guard<std::mutex> lk(g_smu);
    if (!qs || !ad || nseq <= 0) return set_error("bench: bad arguments");
    Q6kView v;
    if (resolve_q6k(w, off, rows, blocks, false, &v)) return -1;
    DevTmp q((size_t)nseq * blocks * QK), d((size_t)nseq * blocks * 4), y((size_t)nseq * rows * 4);
    if (!q.p || !d.p || !y.p) return set_error("hipMalloc");
    Acts a;
    if (h2d(q.p, qs, (size_t)nseq * blocks * QK) || h2d(d.p, ad, (size_t)nseq * blocks * 4) ||
        prep(q.p, (const float *)d.p, false, nseq, blocks, &a))
        return -1;
    return time_launches([&] { matvec_n(v, a, (float *)y.p, rows, blocks, nseq); }, iters, ms_out,
                         "bench");
}

void head_rope(float *x, const float *w, const float *v, float *kc, float *vc, int n_heads, int hd,
               int kv_dim, size_t cache_stride, const int32_t *pos_p, int pos_stride, int pos_fixed,
               int cache_rows, int nseq, float base, float eps) {
    REFUSE_IF(!x || n_heads <= 0 || hd <= 0 || hd % 2 || hd > 256 || nseq <= 0,
              "rope: n_head %d, head_dim %d (even, at most 256), nseq %d", n_heads, hd, nseq);
    REFUSE_IF(kc && (!vc || !v || kv_dim != n_heads * hd),
              "k_norm_rope_store: kv_dim %d must be n_head_kv * head_dim = %d", kv_dim, n_heads * hd);
    int rows = 0;
    const float *den = nullptr;
    const float2 *cs = rope_table(hd, base, &rows, &den);
    if (!cs) return fwd_refused();
    HeadRopeArgs a{};
    a.x = x;
    a.w = w;
    a.eps = eps;
    a.cs = cs;
    a.cs_rows = rows;
    a.den = den;
    // the cache slice's rows: max_kv (batched), else the rows left in kc's
    // allocation when the library made it, else the default table's length
    a.cache_rows = ROPE_DEFAULT_ROWS;
    if (kc) {
        uintptr_t a0, a1;
        std::lock_guard<std::mutex> lk(g_cmu);
        if (alloc_range((uintptr_t)kc, &a0, &a1))
            a.cache_rows = (int)std::min<size_t>((a1 - (uintptr_t)kc) / ((size_t)kv_dim * sizeof(float)), INT_MAX);
    }
    if (cache_rows > 0) a.cache_rows = cache_rows;
    a.pos_p = pos_p;
    a.pos_stride = pos_stride;
    a.pos_fixed = pos_fixed;
    a.n_heads = n_heads;
    a.hd = hd;
    a.kc = kc;
    a.vc = vc;
    a.v = v;
    a.kv_dim = kv_dim;
    a.cache_seq_stride = cache_stride;
    if (launch_head_norm_rope(a, nseq, S())) REFUSE("rope: launch");
}

void attend(const float *q, const float *kc, const float *vc, float *out, int n_head, int n_head_kv,
            int hd, const int32_t *pos, int pos_stride, int n_kv, int max_kv, int nseq) {
    REFUSE_IF(!q || !kc || !vc || !out || n_head_kv <= 0 || n_head % n_head_kv || hd % 4 ||
                  hd <= 0 || hd > 256 || nseq <= 0,
              "attention: n_head %d, n_head_kv %d, head_dim %d", n_head, n_head_kv, hd);
    REFUSE_IF(max_kv > attend_max_kv() || n_kv > attend_max_kv(),
              "attention: at most %d positions (asked %d)", attend_max_kv(), std::max(max_kv, n_kv));
    const float scale = 1.0f / sqrtf((float)hd);  // attention.rs:87
    if (launch_attend_decode(q, kc, vc, pos, n_head, n_head_kv, hd, scale, out, S(), nseq, n_kv,
                             pos_stride, (size_t)max_kv * n_head_kv * hd))
        REFUSE("attention: launch");
}

void embed(const void *table, const int32_t *tok, int tok_stride, int token, float *out, int blocks,
           int nseq) {
    REFUSE_IF(!table || !out || blocks <= 0 || nseq <= 0, "embed: bad arguments");
    if (!tok) {
        uintptr_t a0, a1;
        std::lock_guard<std::mutex> lk(g_cmu);
        const uintptr_t p = (uintptr_t)table;
        const size_t rowb = (size_t)blocks * 210;
        REFUSE_IF(token < 0 || (alloc_range(p, &a0, &a1) && (size_t)token >= (a1 - p) / rowb),
                  "embed: token %d outside the table", token);
    }
    if (launch_embed_q6k(table, tok, blocks, out, S(), nseq, tok_stride, token))
        REFUSE("embed: launch");
}

}  // namespace

// ---- the device-memory bookkeeping behind resolve_q6k ------------------------
void llamd::note_alloc(void *p, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_cmu);
    g_alloc[(uintptr_t)p] = bytes;
}

void llamd::note_free(void *p) {
    std::lock_guard<std::mutex> lk(g_cmu);
    auto it = g_alloc.find((uintptr_t)p);
    if (it == g_alloc.end()) return;
    const uintptr_t a0 = it->first, a1 = it->first + it->second;
    g_alloc.erase(it);
    for (size_t i = 0; i < g_shadow.size();) {
        if (g_shadow[i].lo >= a0 && g_shadow[i].lo < a1) {
            (void)hipFree(g_shadow[i].tiled);
            g_shadow.erase(g_shadow.begin() + i);
        } else {
            ++i;
        }
    }
}

int llamd::note_write(const void *p, size_t bytes, hipStream_t st) {
    std::lock_guard<std::mutex> lk(g_cmu);
    const uintptr_t w0 = (uintptr_t)p, w1 = w0 + bytes;
    for (auto &sh : g_shadow)
        if (sh.lo < w1 && w0 < sh.hi && launch_q6k_retile(sh.src, sh.rows, sh.blocks, sh.tiled, st))
            return set_error("re-tiling after a write: launch failed");
    return 0;
}

int llamd::shadow_q6k(const void *w, const size_t *off, int rows, int blocks, const void **tiled,
                      int *rows_total) {
    std::lock_guard<std::mutex> lk(g_cmu);
    const uintptr_t p = (uintptr_t)w;
    const bool planar = off != nullptr;
    for (auto &sh : g_shadow)
        if (sh.key == p && sh.planar == planar && sh.blocks == blocks &&
            (!planar || !memcmp(sh.off, off, sizeof sh.off))) {
            *tiled = sh.tiled;
            *rows_total = sh.rows;
            return 0;
        }
    uintptr_t a0, a1;
    if (!alloc_range(p, &a0, &a1))
        return set_error("Q6_K weight %p is neither a tiled upload (llamd_rocm_upload_q6k) nor in "
                         "memory from llamd_fwd_alloc / llamd_rocm_upload", w);
    Shadow sh{};
    sh.key = p;
    sh.planar = planar;
    sh.blocks = blocks;
    sh.src.base = (const uint8_t *)w;
    size_t total = 0;
    if (!planar) {
        // ggml blocks, row after row (crates/llamd-quant/src/lib.rs:171-177)
        const size_t rowb = (size_t)blocks * 210;
        total = (a1 - p) / rowb;
        const size_t o[4] = {0, 128, 192, 208};
        for (int f = 0; f < 4; ++f) {
            sh.src.off[f] = o[f];
            sh.src.stride[f] = 210;
        }
        sh.lo = p;
        sh.hi = p + total * rowb;
    } else {
        // PlanarQ6K::layout (crates/llamd-quant/src/dot.rs:349-398): planes
        // of 128, 64, 16 and 2 bytes per block
        memcpy(sh.off, off, sizeof sh.off);
        const size_t fs[4] = {128, 64, 16, 2};
        if (off[1] <= off[0] || (off[1] - off[0]) % 128)
            return set_error("planar offsets: the ql plane is not a whole number of blocks");
        const size_t n = (off[1] - off[0]) / 128;
        if (off[2] - off[1] != 64 * n || off[3] - off[2] != 16 * n)
            return set_error("planar offsets do not describe %zu blocks", n);
        if (n % blocks) return set_error("planar: %zu blocks is not a whole number of rows", n);
        total = n / blocks;
        for (int f = 0; f < 4; ++f) {
            sh.src.off[f] = off[f];
            sh.src.stride[f] = fs[f];
        }
        sh.lo = p + off[0];
        sh.hi = p + off[3] + 2 * n;
        if (sh.hi > a1) return set_error("planar tensor runs past its allocation");
    }
    if (total < (size_t)rows || total > (size_t)INT_MAX)
        return set_error("Q6_K weight holds %zu rows of %d blocks, %d asked", total, blocks, rows);
    sh.rows = (int)total;
    const size_t bytes = llamd_hip_q6k_tiled_bytes(sh.rows, blocks);
    if (hipMalloc(&sh.tiled, bytes) != hipSuccess)
        return set_error("tiled copy: hipMalloc of %zu bytes", bytes);
    // inside a capture the copy is made outside the graph, on a side stream
    hipStream_t st = S();
    const bool cap = capturing(st);
    if (cap) st = side();
    if (!st || launch_q6k_retile(sh.src, sh.rows, blocks, sh.tiled, st) ||
        (cap && hipStreamSynchronize(st) != hipSuccess)) {
        (void)hipFree(sh.tiled);
        return set_error("tiled copy: re-tiling failed");
    }
    g_shadow.push_back(sh);
    *tiled = sh.tiled;
    *rows_total = sh.rows;
    return 0;
}

extern "C" {

// ---- memory ----------------------------------------------------------------
int llamd_fwd_memset(void *p, int value, size_t bytes) {
    if (!p && bytes) return set_error("memset: null pointer");
    if (launch_fill(p, value, bytes, S())) return set_error("memset: launch");
    return note_write(p, bytes, S());
}

size_t llamd_fwd_free_mem(void) {
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) != hipSuccess) return 0;
    return f;
}

// ---- single-sequence f32 pieces (llamd_forward.hip) ---------------------------
void llamd_fwd_embed(const void *table, int token, float *out, int blocks) {
    embed(table, nullptr, 0, token, out, blocks, 1);
}

void llamd_fwd_embed_meta(const void *table, const int32_t *meta, float *out, int blocks) {
    REFUSE_IF(!meta, "embed_meta: null meta");
    embed(table, meta, 0, 0, out, blocks, 1);
}

void llamd_fwd_rope(float *x, int pos, int n_head, int hd, float freq_base) {
    REFUSE_IF(pos < 0, "rope: position %d", pos);
    head_rope(x, nullptr, nullptr, nullptr, nullptr, n_head, hd, 0, 0, nullptr, 0, pos, 0, 1, freq_base,
              0.0f);
}

void llamd_fwd_norm_rope(float *x, const float *w, int n_head, int hd, const int32_t *meta,
                         float freq_base, float eps) {
    REFUSE_IF(!meta, "norm_rope: null meta");
    head_rope(x, w, nullptr, nullptr, nullptr, n_head, hd, 0, 0, meta + 1, 0, 0, 0, 1, freq_base, eps);
}

void llamd_fwd_k_norm_rope_store(float *k, const float *w, const float *v, float *kc, float *vc,
                                 int n_head_kv, int hd, int kv_dim, const int32_t *meta,
                                 float freq_base, float eps) {
    REFUSE_IF(!meta || !kc, "k_norm_rope_store: null meta or cache");
    head_rope(k, w, v, kc, vc, n_head_kv, hd, kv_dim, 0, meta + 1, 0, 0, 0, 1, freq_base, eps);
}

void llamd_fwd_kv_store(float *kc, float *vc, const float *k, const float *v, int pos, int kv_dim) {
    REFUSE_IF(!kc || !vc || !k || !v || pos < 0 || kv_dim <= 0, "kv_store: bad arguments");
    if (launch_kv_store(kc, vc, k, v, pos, kv_dim, S())) REFUSE("kv_store: launch");
}

void llamd_fwd_attention(const float *q, const float *kc, const float *vc, float *out,
                         float *scores, int n_head, int n_head_kv, int hd, int n_kv) {
    (void)scores;  // the logits stay in LDS
    REFUSE_IF(n_kv <= 0, "attention: n_kv %d", n_kv);
    attend(q, kc, vc, out, n_head, n_head_kv, hd, nullptr, 0, n_kv, 0, 1);
}

void llamd_fwd_attention_meta(const float *q, const float *kc, const float *vc, float *out,
                              float *scores, int n_head, int n_head_kv, int hd, const int32_t *meta,
                              int max_kv) {
    (void)scores;
    REFUSE_IF(!meta, "attention_meta: null meta");
    attend(q, kc, vc, out, n_head, n_head_kv, hd, meta + 1, 0, 0, max_kv, 1);
}

void llamd_fwd_add(const float *a, const float *b, float *out, int n) {
    REFUSE_IF(!a || !b || !out || n < 0, "add: bad arguments");
    if (launch_ew(EW_ADD, a, b, 0.0f, out, (size_t)n, S())) REFUSE("add: launch");
}

// ---- Q6_K: ggml blocks, split-k spellings, planar ------------------------------
void llamd_fwd_matvec_splitk(const void *d_w, const int8_t *d_aq, const float *d_ad, float *d_out,
                             int blocks, int rows, int nsub) {
    (void)nsub;  // the K split is chosen by the library
    matvec_entry(d_w, nullptr, d_aq, d_ad, false, d_out, blocks, rows, 1);
}

int llamd_rocm_splitk_bench(const void *d_w, const int8_t *aq, const float *ad, int blocks,
                            int rows, int nsub, int iters, float *ms_out) {
    (void)nsub;
    return bench_matvec(d_w, nullptr, aq, ad, blocks, rows, 1, iters, ms_out);
}

void llamd_fwd_planar_matvec(const void *base, const size_t *off, const int8_t *d_aq,
                             const float *d_ad, float *d_out, int blocks, int rows) {
    REFUSE_IF(!off, "planar: null offsets");
    matvec_entry(base, off, d_aq, d_ad, false, d_out, blocks, rows, 1);
}

void llamd_fwd_planar_grouped(const void *base, const size_t *off, const int32_t *d_ids,
                              const int8_t *d_aq, const float *d_ad, float *d_out, int blocks,
                              int rows, int n_used) {
    REFUSE_IF(!off, "planar: null offsets");
    grouped_entry(base, off, d_ids, d_aq, d_ad, d_out, blocks, rows, n_used);
}

void llamd_fwd_planar_grouped_pa(const void *base, const size_t *off, const int32_t *d_ids,
                                 const int8_t *d_aq, const float *d_ad, float *d_out, int blocks,
                                 int rows, int n_used) {
    REFUSE_IF(!off, "planar: null offsets");
    grouped_pa_entry(base, off, d_ids, d_aq, d_ad, false, d_out, blocks, rows, n_used, 1);
}

void llamd_fwd_planar_x3(const void *b0, const size_t *f0, const void *b1, const size_t *f1,
                         const void *b2, const size_t *f2, const int8_t *d_aq, const float *d_ad,
                         float *o0, float *o1, float *o2, int blocks, int rows0, int rows1,
                         int rows2) {
    REFUSE_IF(!f0 || !f1 || !f2, "planar: null offsets");
    const void *w[3] = {b0, b1, b2};
    const size_t *f[3] = {f0, f1, f2};
    float *o[3] = {o0, o1, o2};
    const int r[3] = {rows0, rows1, rows2};
    x3_entry(w, f, d_aq, d_ad, false, o, blocks, r, 1);
}

void llamd_fwd_planar_grouped_x2(const void *ba, const size_t *fa, const void *bb, const size_t *fb,
                                 const int32_t *d_ids, const int8_t *d_aq, const float *d_ad,
                                 float *oa, float *ob, int blocks, int rows, int n_used) {
    REFUSE_IF(!fa || !fb, "planar: null offsets");
    grouped_x2_entry(ba, fa, bb, fb, d_ids, d_aq, d_ad, false, oa, ob, blocks, rows, n_used, 1);
}

int llamd_rocm_planar_matvec(const void *base, const size_t *off, const int8_t *aq,
                             const float *ad, float *out, int blocks, int rows) {
    if (!off) return set_error("planar: null offsets");
    return host_matvec(base, off, aq, ad, out, blocks, rows, 1);
}

int llamd_rocm_planar_bench(const void *base, const size_t *off, const int8_t *aq, const float *ad,
                            int blocks, int rows, int iters, float *ms_out) {
    if (!off) return set_error("planar: null offsets");
    return bench_matvec(base, off, aq, ad, blocks, rows, 1, iters, ms_out);
}

// ---- batched decode (llamd_batch.hip) -------------------------------------------
// Sequences per batched call: one token chunk of the batched MFMA kernel.
int llamd_batch_max_seq(void) { return CHUNK; }

void llamd_b_embed(const void *table, const int32_t *meta, float *out, int blocks, int nseq) {
    REFUSE_IF(!meta, "b_embed: null meta");
    embed(table, meta, 2, 0, out, blocks, nseq);
}

void llamd_b_rms_norm_quant(const float *x, const float *w, float *out, int8_t *qs, float *d,
                            float *inv, int n, int nseq, float eps) {
    REFUSE_IF(!x || !w || !qs || !d || nseq <= 0, "b_rms_norm_quant: bad arguments");
    if (launch_rms_norm_quant(x, w, out, qs, d, inv, n, eps, S(), nseq))
        REFUSE("b_rms_norm_quant: n must be a multiple of 256, at most 8192");
}

void llamd_b_rms_norm_mul(const float *x, const float *w, float *out, int n, int nseq, float eps) {
    REFUSE_IF(!x || !w || !out || nseq <= 0, "b_rms_norm_mul: bad arguments");
    if (launch_rms_norm_mul(x, w, out, nseq, n, n, eps, S()))
        REFUSE("b_rms_norm_mul: n must be in 1..8192");
}

void llamd_b_quantize(const float *x, int8_t *qs, float *d, int nblocks) {
    REFUSE_IF(!x || !qs || !d || nblocks <= 0, "b_quantize: bad arguments");
    if (launch_q8k_quantize(x, qs, d, nullptr, nblocks, S())) REFUSE("b_quantize: launch");
}

void llamd_b_matvec(const void *w, const int8_t *aq, const float *ad, float *out, int blocks,
                    int rows, int nseq) {
    matvec_entry(w, nullptr, aq, ad, false, out, blocks, rows, nseq);
}

void llamd_b_matvec_x3(const void *w0, const void *w1, const void *w2, const int8_t *aq,
                       const float *ad, float *o0, float *o1, float *o2, int blocks, int r0, int r1,
                       int r2, int nseq) {
    const void *w[3] = {w0, w1, w2};
    const size_t *f[3] = {nullptr, nullptr, nullptr};
    float *o[3] = {o0, o1, o2};
    const int r[3] = {r0, r1, r2};
    x3_entry(w, f, aq, ad, false, o, blocks, r, nseq);
}

void llamd_b_grouped_x2(const void *wa, const void *wb, const int32_t *ids, const int8_t *aq,
                        const float *ad, float *oa, float *ob, int blocks, int rows, int n_used,
                        int nseq) {
    grouped_x2_entry(wa, nullptr, wb, nullptr, ids, aq, ad, false, oa, ob, blocks, rows, n_used, nseq);
}

void llamd_b_grouped_pa(const void *w, const int32_t *ids, const int8_t *aq, const float *ad,
                        float *out, int blocks, int rows, int n_used, int nseq) {
    grouped_pa_entry(w, nullptr, ids, aq, ad, false, out, blocks, rows, n_used, nseq);
}

void llamd_b_norm_rope(float *x, const float *w, int n_head, int hd, const int32_t *meta, int nseq,
                       float freq_base, float eps) {
    REFUSE_IF(!meta, "b_norm_rope: null meta");
    head_rope(x, w, nullptr, nullptr, nullptr, n_head, hd, 0, 0, meta + 1, 2, 0, 0, nseq, freq_base,
              eps);
}

void llamd_b_k_norm_rope_store(float *k, const float *w, const float *v, float *kc, float *vc,
                               int n_head_kv, int hd, int kv_dim, int max_kv, const int32_t *meta,
                               int nseq, float freq_base, float eps) {
    REFUSE_IF(!meta || !kc || max_kv <= 0, "b_k_norm_rope_store: bad arguments");
    head_rope(k, w, v, kc, vc, n_head_kv, hd, kv_dim, (size_t)max_kv * kv_dim, meta + 1, 2, 0,
              max_kv, nseq, freq_base, eps);
}

void llamd_b_attention(const float *q, const float *kc, const float *vc, float *out, float *scores,
                       int n_head, int n_head_kv, int hd, int max_kv, const int32_t *meta,
                       int nseq) {
    (void)scores;
    REFUSE_IF(!meta || max_kv <= 0, "b_attention: bad arguments");
    attend(q, kc, vc, out, n_head, n_head_kv, hd, meta + 1, 2, 0, max_kv, nseq);
}

void llamd_b_add(const float *a, const float *b, float *o, int n) { llamd_fwd_add(a, b, o, n); }

void llamd_b_silu_mul(const float *g, const float *u, float *o, int n) {
    REFUSE_IF(!g || !u || !o || n < 0, "b_silu_mul: bad arguments");
    if (launch_silu_mul(g, u, o, n, S())) REFUSE("b_silu_mul: launch");
}

void llamd_b_matvec_f32(const float *w, const float *x, float *out, int k, int rows, int nseq) {
    REFUSE_IF(!w || !x || !out || k <= 0 || rows <= 0 || nseq <= 0, "b_matvec_f32: bad arguments");
    if (launch_matvec_f32_exact(w, x, out, rows, k, nseq, S())) REFUSE("b_matvec_f32: launch");
}

void llamd_b_router(const float *logits, int n_expert, int n_used, int32_t *ids, float *weights,
                    float *probs, int nseq) {
    REFUSE_IF(!logits || !ids || !weights || nseq <= 0 || n_expert <= 0 || n_expert > 256 ||
                  n_used <= 0 || n_used > n_expert,
              "b_router: n_expert %d (at most 256), n_used %d, nseq %d", n_expert, n_used, nseq);
    if (launch_route_logits(logits, n_expert, n_used, ids, weights, S(), nseq, probs))
        REFUSE("b_router: launch");
}

void llamd_b_moe_combine_add(const float *down, const float *weights, const float *residual,
                             float *out, int n_used, int n_embd, int nseq) {
    REFUSE_IF(!down || !weights || !residual || !out || n_used <= 0 || n_embd <= 0 || nseq <= 0,
              "b_moe_combine_add: bad arguments");
    if (launch_moe_combine(down, weights, residual, out, n_used, n_embd, nseq, S()))
        REFUSE("b_moe_combine_add: launch");
}

void llamd_b_argmax(const float *x, int n, float *sv, int32_t *si, int32_t *out, int nchunk,
                    int nseq) {
    REFUSE_IF(!x || !sv || !si || !out || n <= 0 || nchunk <= 0 || nseq <= 0,
              "b_argmax: bad arguments");
    if (launch_argmax(x, n, n, nseq, sv, (int *)si, out, S(), nchunk)) REFUSE("b_argmax: launch");
}

// ---- unsigned-activation form (llamd_udot.hip) ------------------------------------
void llamd_u_set_tile(int t) { g_u_tile = (t == 2 || t == 4) ? t : 1; }
int llamd_u_get_tile(void) { return g_u_tile; }

void llamd_u_bias_sums(const int8_t *qs, uint8_t *qb, int32_t *sb, int nblocks) {
    REFUSE_IF(!qs || !qb || !sb || nblocks <= 0, "u_bias_sums: bad arguments");
    if (launch_bias_sums(qs, qb, sb, nblocks, S())) REFUSE("u_bias_sums: launch");
}

void llamd_u_quantize(const float *x, uint8_t *qb, int32_t *sb, float *d, int nblocks) {
    REFUSE_IF(!x || !qb || !sb || !d || nblocks <= 0, "u_quantize: bad arguments");
    // signed Q8_K into qb, then biased in place
    if (launch_q8k_quantize(x, (int8_t *)qb, d, nullptr, nblocks, S()) ||
        launch_bias_sums((const int8_t *)qb, qb, sb, nblocks, S()))
        REFUSE("u_quantize: launch");
}

void llamd_u_norm_quant(const float *x, const float *w, float *out, uint8_t *qb, int32_t *sb,
                        float *d, float *inv, int n, int nseq, float eps) {
    REFUSE_IF(!x || !w || !qb || !sb || !d || nseq <= 0 || n <= 0 || n % QK,
              "u_norm_quant: bad arguments");
    if (launch_rms_norm_quant(x, w, out, (int8_t *)qb, d, inv, n, eps, S(), nseq) ||
        launch_bias_sums((const int8_t *)qb, qb, sb, nseq * (n / QK), S()))
        REFUSE("u_norm_quant: n must be a multiple of 256, at most 8192");
}

void llamd_u_matvec(const void *base, const size_t *off, const uint8_t *qb, const int32_t *sb,
                    const float *ad, float *out, int blocks, int rows, int nseq) {
    (void)sb;
    REFUSE_IF(!off, "u_matvec: null offsets");
    matvec_entry(base, off, qb, ad, true, out, blocks, rows, nseq);
}

void llamd_u_x3(const void *b0, const size_t *f0, const void *b1, const size_t *f1, const void *b2,
                const size_t *f2, const uint8_t *qb, const int32_t *sb, const float *ad, float *o0,
                float *o1, float *o2, int blocks, int r0, int r1, int r2, int nseq) {
    (void)sb;
    REFUSE_IF(!f0 || !f1 || !f2, "u_x3: null offsets");
    const void *w[3] = {b0, b1, b2};
    const size_t *f[3] = {f0, f1, f2};
    float *o[3] = {o0, o1, o2};
    const int r[3] = {r0, r1, r2};
    x3_entry(w, f, qb, ad, true, o, blocks, r, nseq);
}

void llamd_u_grouped_x2(const void *ba, const size_t *fa, const void *bb, const size_t *fb,
                        const int32_t *ids, const uint8_t *qb, const int32_t *sb, const float *ad,
                        float *oa, float *ob, int blocks, int rows, int n_used, int nseq) {
    (void)sb;
    REFUSE_IF(!fa || !fb, "u_grouped_x2: null offsets");
    grouped_x2_entry(ba, fa, bb, fb, ids, qb, ad, true, oa, ob, blocks, rows, n_used, nseq);
}

void llamd_u_grouped_pa(const void *base, const size_t *off, const int32_t *ids, const uint8_t *qb,
                        const int32_t *sb, const float *ad, float *out, int blocks, int rows,
                        int n_used, int nseq) {
    (void)sb;
    REFUSE_IF(!off, "u_grouped_pa: null offsets");
    grouped_pa_entry(base, off, ids, qb, ad, true, out, blocks, rows, n_used, nseq);
}

int llamd_u_norm_quant_host(const float *x, const float *w, int n, int nseq, float eps, float *out,
                            uint8_t *qb, int32_t *sb, float *d) {
    if (!x || !w || !out || !qb || !sb || !d || nseq <= 0 || n <= 0 || n % QK)
        return set_error("u_norm_quant_host: bad arguments");
    const int nb = n / QK;
    const size_t xn = (size_t)n * nseq;
    DevTmp dx(xn * 4), dw((size_t)n * 4), dout(xn * 4), dq(xn), ds((size_t)nb * 16 * nseq * 4),
        dd((size_t)nb * nseq * 4), di((size_t)nseq * 4);
    if (!dx.p || !dw.p || !dout.p || !dq.p || !ds.p || !dd.p || !di.p) return set_error("hipMalloc");
    if (h2d(dx.p, x, xn * 4) || h2d(dw.p, w, (size_t)n * 4)) return -1;
    llamd_u_norm_quant((float *)dx.p, (float *)dw.p, (float *)dout.p, (uint8_t *)dq.p,
                       (int32_t *)ds.p, (float *)dd.p, (float *)di.p, n, nseq, eps);
    if (llamd_fwd_last_error()) return -1;
    if (d2h(out, dout.p, xn * 4) || d2h(qb, dq.p, xn) || d2h(sb, ds.p, (size_t)nb * 16 * nseq * 4) ||
        d2h(d, dd.p, (size_t)nb * nseq * 4))
        return -1;
    return sync_check("u_norm_quant_host");
}

int llamd_u_quantize_host(const float *x, int nblocks, uint8_t *qb, int32_t *sb, float *d) {
    if (!x || !qb || !sb || !d || nblocks <= 0) return set_error("u_quantize_host: bad arguments");
    const size_t n = (size_t)nblocks * QK;
    DevTmp dx(n * 4), dq(n), ds((size_t)nblocks * 64), dd((size_t)nblocks * 4);
    if (!dx.p || !dq.p || !ds.p || !dd.p) return set_error("hipMalloc");
    if (h2d(dx.p, x, n * 4)) return -1;
    llamd_u_quantize((float *)dx.p, (uint8_t *)dq.p, (int32_t *)ds.p, (float *)dd.p, nblocks);
    if (llamd_fwd_last_error()) return -1;
    if (d2h(qb, dq.p, n) || d2h(sb, ds.p, (size_t)nblocks * 64) || d2h(d, dd.p, (size_t)nblocks * 4))
        return -1;
    return sync_check("u_quantize_host");
}

int llamd_u_matvec_host(const void *base, const size_t *off, const int8_t *qs, const float *ad,
                        float *out, int blocks, int rows, int nseq) {
    if (!off) return set_error("u_matvec_host: null offsets");
    return host_matvec(base, off, qs, ad, out, blocks, rows, nseq);
}

int llamd_u_matvec_bench(const void *base, const size_t *off, const int8_t *qs, const float *ad,
                         int blocks, int rows, int nseq, int iters, float *ms_out) {
    if (!off) return set_error("u_matvec_bench: null offsets");
    return bench_matvec(base, off, qs, ad, blocks, rows, nseq, iters, ms_out);
}

// ---- benchmarking -------------------------------------------------------------------
// n Q6_K matvecs (the same checks and launch as llamd_fwd_matvec) enqueued
// from one call, so a timed region of short launches measures the device and
// not the calling language's per-call overhead.
int llamd_hip_matvec_many(const void *const *w, const int8_t *const *aq, const float *const *ad,
                          float *const *out, const int *blocks, const int *rows, int n) {
    if (n < 0 || (n && (!w || !aq || !ad || !out || !blocks || !rows)))
        return set_error("matvec_many: bad arguments");
    for (int i = 0; i < n; ++i) {
        Q6kView v;
        if (resolve_q6k(w[i], nullptr, rows[i], blocks[i], false, &v)) return -1;
        if (launch_q6k_mv_b1(v.tiled, 0, nullptr, aq[i], ad[i], out[i], rows[i], blocks[i], 1, 0, S()))
            return set_error("matvec_many: launch %d failed", i);
    }
    return 0;
}

// ---- llamd-tensor Backend, row-wise (not in the reference's C ABI) ----------------
// CpuBackend (crates/llamd-cpu/src/lib.rs:55-224) on device tensors, with the
// same float operations in the same order: bit-identical results.
int llamd_hip_be_rms_norm(const float *x, float *out, int rows, int n, float eps) {
    if (!x || !out) return set_error("rms_norm: null pointer");
    return launch_rms_norm_mul(x, nullptr, out, rows, n, n, eps, S())
               ? set_error("rms_norm: rows > 0 and n in 1..8192") : 0;
}

int llamd_hip_be_softmax(const float *x, float *out, int rows, int n) {
    if (!x || !out) return set_error("softmax: null pointer");
    return launch_softmax_rows(x, out, rows, n, S()) ? set_error("softmax: rows, n > 0") : 0;
}

int llamd_hip_be_silu(const float *x, float *out, size_t n) {
    if (!x || !out) return set_error("silu: null pointer");
    return launch_ew(EW_SILU, x, nullptr, 0.0f, out, n, S()) ? set_error("silu: launch") : 0;
}

int llamd_hip_be_add(const float *a, const float *b, float *out, size_t n) {
    if (!a || !b || !out) return set_error("add: null pointer");
    return launch_ew(EW_ADD, a, b, 0.0f, out, n, S()) ? set_error("add: launch") : 0;
}

int llamd_hip_be_mul(const float *a, const float *b, float *out, size_t n) {
    if (!a || !b || !out) return set_error("mul: null pointer");
    return launch_ew(EW_MUL, a, b, 0.0f, out, n, S()) ? set_error("mul: launch") : 0;
}

int llamd_hip_be_scale(const float *x, float by, float *out, size_t n) {
    if (!x || !out) return set_error("scale: null pointer");
    return launch_ew(EW_SCALE, x, nullptr, by, out, n, S()) ? set_error("scale: launch") : 0;
}

int llamd_hip_be_matmul(const float *w, const float *x, float *out, int m, int n, int k) {
    if (!w || !x || !out) return set_error("matmul: null pointer");
    return launch_matmul_f32_seq(w, x, out, m, n, k, S())
               ? set_error("matmul: m, k > 0 and n in 1..65535") : 0;
}

int llamd_hip_be_rope(float *x, int rows, int row_len, const uint32_t *positions, int head_dim,
                      float freq_base, float freq_scale) {
    if (!x || !positions || rows <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 256 ||
        row_len % head_dim)
        return set_error("rope: head_dim %d (even, at most 256) must divide the row length %d",
                         head_dim, row_len);
    // one table row per tensor row, at that row's own position * freq_scale
    const int half = head_dim / 2;
    std::vector<float> den(half);
    for (int i = 0; i < half; ++i) den[i] = powf(freq_base, 2.0f * (float)i / (float)head_dim);
    std::vector<float2> cs((size_t)rows * half);
    for (int r = 0; r < rows; ++r) {
        const float pos = (float)positions[r] * freq_scale;
        for (int i = 0; i < half; ++i) {
            const float theta = pos / den[i];
            cs[(size_t)r * half + i] = make_float2(cosf(theta), sinf(theta));
        }
    }
    DevTmp t(cs.size() * sizeof(float2));
    if (!t.p) return set_error("hipMalloc");
    if (h2d(t.p, cs.data(), cs.size() * sizeof(float2))) return -1;
    HeadRopeArgs a{};
    a.x = x;
    a.cs = (const float2 *)t.p;
    a.cs_rows = rows;
    a.pos_fixed = -1;  // row s reads table row s
    a.n_heads = row_len / head_dim;
    a.hd = head_dim;
    if (launch_head_norm_rope(a, rows, S())) return set_error("rope: launch");
    return sync_check("rope");  // the table is freed on return
}

int llamd_hip_be_get_rows(const float *table, int table_rows, int row_len, const uint32_t *ids,
                          int n_ids, float *out) {
    if (!table || !out || !ids || row_len <= 0 || n_ids < 0) return set_error("get_rows: bad arguments");
    for (int j = 0; j < n_ids; ++j) {
        if (ids[j] >= (uint32_t)table_rows)
            return set_error("get_rows: id %u is outside a table of %d rows", ids[j], table_rows);
        if (hipMemcpyAsync(out + (size_t)j * row_len, table + (size_t)ids[j] * row_len,
                           (size_t)row_len * 4, hipMemcpyDeviceToDevice, S()) != hipSuccess)
            return set_error("get_rows: copy failed");
    }
    return 0;
}

}  // extern "C"
