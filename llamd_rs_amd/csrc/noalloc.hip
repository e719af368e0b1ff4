// noalloc.hip -- the LM-head call (Q6_K matvec over the vocabulary + argmax)
// for callers that cannot allocate device memory: code being captured into a
// HIP graph, serving loops, harnesses that forbid hipMalloc.
//
// llamd_hip_lmhead_forward keeps its scratch (Q8_K of x, per-tile arg-max
// candidates) in buffers allocated at llamd_hip_lmhead_create. This entry
// point runs the same launches (lmhead_enqueue, capi.cpp) with that scratch
// carved from one file-scope device array instead, so a call allocates
// nothing: no hipMalloc, no hipFree, no allocating library routine.
//
// The array is a module-scope __device__ object: every GPU the library runs
// on holds its own copy, for the life of the process. Host code never uses
// the array's name as an address (on the host it names a stand-in, not
// device memory): the device address is taken once per device with
// hipGetSymbolAddress and kept, and only that address reaches a kernel.
//
// Every call on one GPU shares that GPU's array and leaves its contents
// behind. Nothing in it needs to start at zero (every tile writes its
// candidate, the quantizer writes every block), so nothing is cleared; two
// calls that overlap on one GPU (two host threads, two streams) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/llamd_hip.h"
#include "errors.hpp"
#include "launch.hpp"

namespace {

constexpr int QK = 256;
// Limits of one call: vocabulary rows, 256-blocks per row (k <= 8192) and
// sequences.
constexpr int NA_MAX_ROWS = 262144;
constexpr int NA_MAX_BLOCKS = 32;
constexpr int NA_MAX_SEQ = 16;
constexpr size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
constexpr size_t NA_TILES = NA_MAX_ROWS / 16;
constexpr size_t NA_XQ = align256((size_t)NA_MAX_BLOCKS * QK);           // nseq == 1
constexpr size_t NA_XD = align256((size_t)NA_MAX_BLOCKS * 4);
constexpr size_t NA_CQ = align256((size_t)NA_MAX_BLOCKS * 4096);         // one 16-token chunk
constexpr size_t NA_CD = align256((size_t)NA_MAX_BLOCKS * 16 * 4);
constexpr size_t NA_PV = align256(NA_TILES * NA_MAX_SEQ * 4);
constexpr size_t NA_PI = align256(NA_TILES * NA_MAX_SEQ * 4);
constexpr size_t NA_BYTES = NA_XQ + NA_XD + NA_CQ + NA_CD + NA_PV + NA_PI;  // about 2.3 MB

__device__ __align__(256) unsigned char scratch[NA_BYTES];

constexpr int NA_MAX_DEVICES = 64;
std::mutex g_na_mu;
unsigned char *g_na_ptr[NA_MAX_DEVICES];  // device address of `scratch` per device

// The calling thread's current device's copy of `scratch`, looked up once.
unsigned char *scratch_ptr() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NA_MAX_DEVICES) {
        llamd::set_error("lmhead_forward_noalloc: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (!g_na_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            llamd::set_error("lmhead_forward_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_na_ptr[dev] = (unsigned char *)p;
    }
    return g_na_ptr[dev];
}

}  // namespace

extern "C" {

size_t llamd_hip_lmhead_noalloc_scratch_bytes(void) { return NA_BYTES; }

int llamd_hip_lmhead_forward_noalloc(const void *d_w, int rows, int blocks, const float *d_x,
                                     int nseq, float *d_logits, int32_t *d_ids) {
    int wr = 0, wb = 0, ne = 0;
    if (!d_w || llamd::q6k_handle_shape(d_w, &wr, &wb, &ne) || ne != 1 || wr != rows || wb != blocks)
        return llamd::set_error("lmhead_forward_noalloc: weight handle does not match rows=%d blocks=%d",
                                rows, blocks);
    if (!d_x || !d_logits || !d_ids || nseq <= 0)
        return llamd::set_error("lmhead_forward_noalloc: bad arguments");
    if (rows > NA_MAX_ROWS || blocks > NA_MAX_BLOCKS || nseq > NA_MAX_SEQ)
        return llamd::set_error("lmhead_forward_noalloc: at most %d rows, %d blocks (k = %d) and %d "
                                "sequences; got rows=%d blocks=%d nseq=%d",
                                NA_MAX_ROWS, NA_MAX_BLOCKS, NA_MAX_BLOCKS * QK, NA_MAX_SEQ, rows,
                                blocks, nseq);
    unsigned char *base = scratch_ptr();
    if (!base) return -1;
    // the kernels index the candidates as [nseq][tiles]: within NA_PV for
    // tiles <= NA_TILES, nseq <= NA_MAX_SEQ; one 16-token chunk holds nseq
    llamd::LmHeadScratch sc;
    sc.xq = (int8_t *)base;
    sc.xd = (float *)(base + NA_XQ);
    sc.cq = (int8_t *)(base + NA_XQ + NA_XD);
    sc.cd = (float *)(base + NA_XQ + NA_XD + NA_CQ);
    sc.pv = (float *)(base + NA_XQ + NA_XD + NA_CQ + NA_CD);
    sc.pi = (int *)(base + NA_XQ + NA_XD + NA_CQ + NA_CD + NA_PV);
    if (llamd::lmhead_chunk_q_bytes(nseq, blocks) > NA_CQ ||
        llamd::lmhead_chunk_d_bytes(nseq, blocks) > NA_CD)
        return llamd::set_error("lmhead_forward_noalloc: internal scratch layout too small");
    return llamd::lmhead_enqueue(d_w, rows, blocks, d_x, nseq, d_logits, d_ids, sc)
               ? llamd::set_error("lmhead_forward_noalloc: launch failed")
               : 0;
}

}  // extern "C"
