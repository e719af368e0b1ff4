// layout.cpp -- host-side weight layouts for the gfx950 kernels.
//
// TILED Q6_K. ggml stores Q6_K as 210-byte blocks, row after row
// (crates/llamd-quant/src/lib.rs:171-177): block b of row r sits at
// (r * blocks + b) * 210, which is only 2-byte aligned, and the bytes of one
// weight are spread over three places (low nibble in ql, high bits in qh,
// scale in sc). The matvec kernels instead read, per wave, one segment of 16
// rows x 1 block = 3360 bytes with three fully coalesced 16-byte loads per
// lane. This file defines that segment and converts to and from it. The
// conversion is a pure permutation of bits: every 6-bit code, scale byte and
// f16 d of the input appears exactly once in the output, and
// llamd_hip_q6k_untile() restores the ggml bytes (tests/test_layout.py).
//
// Segment (tile t of 16 rows, block b) lives at byte (t * blocks + b) * 3360.
// Inside it, lane L = n + 16 s (row n = 0..15 of the tile, s = 0..3) owns the
// codes of weights e = 8 m + c for every class c = e mod 8 (the reference's
// eight accumulation lanes, dot.rs:174-193) and m = 8 s .. 8 s + 7:
//   [   0, 1024)  16 B per lane: nibble words N_c, c = 0..3
//   [1024, 2048)  16 B per lane: nibble words N_c, c = 4..7
//                 N_c byte j = lo4(code(c, 8s+j)) | lo4(code(c, 8s+j+4)) << 4
//   [2048, 3072)  16 B per lane: high-bit words H_p, p = 0..3, byte j =
//                 hi2(2p, 8s+j) | hi2(2p, 8s+j+4) << 2
//                 | hi2(2p+1, 8s+j) << 4 | hi2(2p+1, 8s+j+4) << 6
//   [3072, 3328)  4 B per lane: sc[4s .. 4s+3] of row n (the 4 groups of 16
//                 whose weights lane L holds for each class)
//   [3328, 3360)  f16 d of rows 0..15
// Rows past the end of the matrix are zero (d = 0, so they contribute 0).
//
// Q8_0 PLANES. Q8_0 blocks are 34 bytes (2-byte aligned). The device copy
// splits them into a plane of int8 quants [rows][k] followed by a plane of
// f16 scales [rows][k/32]; again a permutation.
#include <stdint.h>
#include <string.h>

#include <vector>

namespace {

constexpr int QK_K = 256;
constexpr int BB = 210;
constexpr int SEG = 16 * BB;

inline int code6(const uint8_t *blk, int e) {
    const int h = e / 128, i = e % 128, q4 = i / 32, l = i % 32;
    const int lo = (blk[h * 64 + l + (q4 & 1) * 32] >> (4 * (q4 >> 1))) & 0xF;
    const int hi = (blk[128 + h * 32 + l] >> (2 * q4)) & 3;
    return lo | (hi << 4);
}

inline void set_code6(uint8_t *blk, int e, int code) {
    const int h = e / 128, i = e % 128, q4 = i / 32, l = i % 32;
    uint8_t &ql = blk[h * 64 + l + (q4 & 1) * 32];
    const int sh = 4 * (q4 >> 1);
    ql = (uint8_t)((ql & ~(0xF << sh)) | ((code & 0xF) << sh));
    uint8_t &qh = blk[128 + h * 32 + l];
    const int sh2 = 2 * q4;
    qh = (uint8_t)((qh & ~(3 << sh2)) | (((code >> 4) & 3) << sh2));
}

inline int elem(int c, int m) { return 8 * m + c; }

void tile_segment(const uint8_t *const rows_blk[16], uint8_t *seg) {
    static const uint8_t zero[BB] = {0};
    memset(seg, 0, SEG);
    for (int n = 0; n < 16; ++n) {
        const uint8_t *blk = rows_blk[n] ? rows_blk[n] : zero;
        for (int s = 0; s < 4; ++s) {
            const int L = n + 16 * s;
            for (int c = 0; c < 8; ++c) {
                for (int j = 0; j < 4; ++j) {
                    const int a = code6(blk, elem(c, 8 * s + j)) & 0xF;
                    const int b = code6(blk, elem(c, 8 * s + j + 4)) & 0xF;
                    seg[(c / 4) * 1024 + 16 * L + 4 * (c % 4) + j] = (uint8_t)(a | (b << 4));
                }
            }
            for (int p = 0; p < 4; ++p) {
                for (int j = 0; j < 4; ++j) {
                    const int h0 = code6(blk, elem(2 * p, 8 * s + j)) >> 4;
                    const int h1 = code6(blk, elem(2 * p, 8 * s + j + 4)) >> 4;
                    const int h2 = code6(blk, elem(2 * p + 1, 8 * s + j)) >> 4;
                    const int h3 = code6(blk, elem(2 * p + 1, 8 * s + j + 4)) >> 4;
                    seg[2048 + 16 * L + 4 * p + j] = (uint8_t)(h0 | (h1 << 2) | (h2 << 4) | (h3 << 6));
                }
            }
            for (int v = 0; v < 4; ++v) seg[3072 + 4 * L + v] = blk[192 + 4 * s + v];
        }
        seg[3328 + 2 * n] = blk[208];
        seg[3328 + 2 * n + 1] = blk[209];
    }
}

void untile_segment(const uint8_t *seg, uint8_t *const rows_blk[16]) {
    for (int n = 0; n < 16; ++n) {
        uint8_t *blk = rows_blk[n];
        if (!blk) continue;
        memset(blk, 0, BB);
        for (int s = 0; s < 4; ++s) {
            const int L = n + 16 * s;
            for (int c = 0; c < 8; ++c) {
                for (int j = 0; j < 4; ++j) {
                    const uint8_t nb = seg[(c / 4) * 1024 + 16 * L + 4 * (c % 4) + j];
                    const uint8_t hb = seg[2048 + 16 * L + 4 * (c / 2) + j];
                    const int hs = (c & 1) ? 4 : 0;
                    const int lo_a = nb & 0xF, lo_b = nb >> 4;
                    const int hi_a = (hb >> hs) & 3, hi_b = (hb >> (hs + 2)) & 3;
                    set_code6(blk, elem(c, 8 * s + j), lo_a | (hi_a << 4));
                    set_code6(blk, elem(c, 8 * s + j + 4), lo_b | (hi_b << 4));
                }
            }
            for (int v = 0; v < 4; ++v) blk[192 + 4 * s + v] = seg[3072 + 4 * L + v];
        }
        blk[208] = seg[3328 + 2 * n];
        blk[209] = seg[3328 + 2 * n + 1];
    }
}

}  // namespace

extern "C" {

size_t llamd_hip_q6k_tiled_bytes(int rows, int blocks) {
    if (rows <= 0 || blocks <= 0) return 0;
    const size_t tiles = ((size_t)rows + 15) / 16;
    return tiles * (size_t)blocks * SEG;
}

// ggml Q6_K bytes [rows][blocks*210] -> tiled layout (llamd_hip_q6k_tiled_bytes).
int llamd_hip_q6k_tile(const void *ggml, int rows, int blocks, void *out) {
    if (!ggml || !out || rows <= 0 || blocks <= 0) return -1;
    const uint8_t *src = (const uint8_t *)ggml;
    uint8_t *dst = (uint8_t *)out;
    const int tiles = (rows + 15) / 16;
    for (int t = 0; t < tiles; ++t) {
        for (int b = 0; b < blocks; ++b) {
            const uint8_t *rb[16];
            for (int n = 0; n < 16; ++n) {
                const int r = 16 * t + n;
                rb[n] = r < rows ? src + ((size_t)r * blocks + b) * BB : nullptr;
            }
            tile_segment(rb, dst + ((size_t)t * blocks + b) * SEG);
        }
    }
    return 0;
}

// Inverse of llamd_hip_q6k_tile (padding rows are dropped).
int llamd_hip_q6k_untile(const void *tiled, int rows, int blocks, void *ggml_out) {
    if (!tiled || !ggml_out || rows <= 0 || blocks <= 0) return -1;
    const uint8_t *src = (const uint8_t *)tiled;
    uint8_t *dst = (uint8_t *)ggml_out;
    const int tiles = (rows + 15) / 16;
    for (int t = 0; t < tiles; ++t) {
        for (int b = 0; b < blocks; ++b) {
            uint8_t *rb[16];
            for (int n = 0; n < 16; ++n) {
                const int r = 16 * t + n;
                rb[n] = r < rows ? dst + ((size_t)r * blocks + b) * BB : nullptr;
            }
            untile_segment(src + ((size_t)t * blocks + b) * SEG, rb);
        }
    }
    return 0;
}

size_t llamd_hip_q8_0_planar_bytes(int rows, int k) {
    if (rows <= 0 || k <= 0 || k % 32) return 0;
    return (size_t)rows * k + (size_t)rows * (k / 32) * 2;
}

// ggml Q8_0 bytes [rows][k/32*34] -> [rows][k] int8 plane + [rows][k/32] f16 plane.
int llamd_hip_q8_0_planarize(const void *ggml, int rows, int k, void *out) {
    if (!ggml || !out || rows <= 0 || k <= 0 || k % 32) return -1;
    const uint8_t *src = (const uint8_t *)ggml;
    uint8_t *qs = (uint8_t *)out;
    uint8_t *dp = qs + (size_t)rows * k;
    const int nb = k / 32;
    for (size_t r = 0; r < (size_t)rows; ++r) {
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = src + (r * nb + b) * 34;
            dp[(r * nb + b) * 2] = blk[0];
            dp[(r * nb + b) * 2 + 1] = blk[1];
            memcpy(qs + r * k + (size_t)b * 32, blk + 2, 32);
        }
    }
    return 0;
}

}  // extern "C"
