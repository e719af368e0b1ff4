// synth.cpp -- seeded synthetic workloads for the benchmark and the tests.
//
// There is no network and no checkpoint: every weight and activation is drawn
// here from a documented generator so the GPU path and the CPU baseline see
// identical bytes.
//
//   SplitMix64 (Steele, Lea & Flood, 2014) -> 53-bit uniform doubles ->
//   Box-Muller -> N(0, sigma) rounded to f32.
//
// The reference has no Q6_K or Q8_0 WEIGHT quantizer (crates/llamd-quant only
// dequantizes; its one quantizer is the Q8_K activation quantizer), so the
// quantizers below are this project's own. They follow ggml's published block
// formats and the simple (non-searching) form of its reference quantizers:
//   Q8_0 : d = amax/127, q = round-half-away(x/d), d stored as f16.
//   Q6_K : per 16-weight group a signed scale max/-32 (the value of largest
//          magnitude maps to code 0, i.e. -32); per 256-block
//          d = max_scale/-128, sc = min(127, nearest(scale/d)); codes
//          q = clamp(nearest(x/(d*sc)) + 32, 0, 63). No make_qx_quants
//          search -- dequantized error is larger than ggml's, which does not
//          matter here: CPU and GPU consume the same bytes, and only the
//          arithmetic on those bytes is under test.
// Their parity is unpinned by construction (nothing in the reference to pin
// them to); tests/test_synth.py checks the format invariants and the
// round-trip error bound instead.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace {

struct SplitMix64 {
    uint64_t s;
    explicit SplitMix64(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    // uniform in (0, 1]
    double unit() { return ((next() >> 11) + 1) * (1.0 / 9007199254740992.0); }
};

uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to inf
    if (ax < 0x38800000u) {                                     // f16 subnormal or zero
        // value = ax as float; f16 subnormal unit is 2^-24
        float a;
        memcpy(&a, &ax, 4);
        const float scaled = a * 16777216.0f;  // exact (power of two)
        const uint32_t m = (uint32_t)nearbyintf(scaled);
        return (uint16_t)(sign | m);
    }
    const uint32_t exp = ((ax >> 23) - 127 + 15);
    uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (exp << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    uint32_t u;
    if (exp == 0x1F) u = sign | 0x7F800000u | (man ? (0x400000u | (man << 13)) : 0);
    else if (exp == 0) {
        if (!man) u = sign;
        else {
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else u = sign | ((exp + 112) << 23) | (man << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

inline int nearest(float v) { return (int)nearbyintf(v); }

void quantize_block_q6k(const float *x, uint8_t *blk) {
    float scales[16];
    for (int g = 0; g < 16; ++g) {
        float amax = 0.f, mx = 0.f;
        for (int i = 0; i < 16; ++i) {
            const float a = fabsf(x[16 * g + i]);
            if (a > amax) { amax = a; mx = x[16 * g + i]; }
        }
        scales[g] = amax > 0.f ? mx / -32.f : 0.f;
    }
    float smax = 0.f, sm = 0.f;
    for (int g = 0; g < 16; ++g)
        if (fabsf(scales[g]) > smax) { smax = fabsf(scales[g]); sm = scales[g]; }
    memset(blk, 0, 210);
    if (smax == 0.f) {
        for (int e = 0; e < 256; ++e) {
            // code 32 = weight 0
            const int h = e / 128, i = e % 128, q4 = i / 32, l = i % 32;
            blk[h * 64 + l + (q4 & 1) * 32] |= (uint8_t)(0 << (4 * (q4 >> 1)));
            blk[128 + h * 32 + l] |= (uint8_t)(2 << (2 * q4));
        }
        return;
    }
    const float iscale = -128.f / sm;
    const uint16_t dh = f32_to_f16_rne(1.f / iscale);
    const float d = f16_to_f32(dh);
    int8_t sc[16];
    for (int g = 0; g < 16; ++g) sc[g] = (int8_t)std::min(127, nearest(iscale * scales[g]));
    for (int g = 0; g < 16; ++g) blk[192 + g] = (uint8_t)sc[g];
    blk[208] = (uint8_t)(dh & 0xFF);
    blk[209] = (uint8_t)(dh >> 8);
    for (int e = 0; e < 256; ++e) {
        const float de = d * (float)sc[e / 16];
        int q = de != 0.f ? nearest(x[e] / de) : 0;
        q = std::max(-32, std::min(31, q)) + 32;
        const int h = e / 128, i = e % 128, q4 = i / 32, l = i % 32;
        blk[h * 64 + l + (q4 & 1) * 32] |= (uint8_t)((q & 0xF) << (4 * (q4 >> 1)));
        blk[128 + h * 32 + l] |= (uint8_t)(((q >> 4) & 3) << (2 * q4));
    }
}

void quantize_block_q8_0(const float *x, uint8_t *blk) {
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, fabsf(x[i]));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    const uint16_t dh = f32_to_f16_rne(d);
    blk[0] = (uint8_t)(dh & 0xFF);
    blk[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 32; ++i) blk[2 + i] = (uint8_t)(int8_t)roundf(x[i] * id);
}

// Row r of a synthetic matrix draws from its own SplitMix64 stream seeded with
// seed ^ (r * golden-ratio constant), so rows can be generated in parallel and
// the result does not depend on the thread count.
template <class Fn>
void for_rows(size_t rows, Fn fn) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (rows < 64) nt = 1;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; ++t)
        th.emplace_back([&, t] {
            for (size_t r = t; r < rows; r += nt) fn(r);
        });
    for (auto &x : th) x.join();
}

void normal_row(uint64_t seed, size_t r, float sigma, float *buf, size_t k) {
    SplitMix64 g(seed ^ ((uint64_t)(r + 1) * 0x9E3779B97F4A7C15ull));
    for (size_t i = 0; i < k; i += 2) {
        const double u1 = g.unit(), u2 = g.unit();
        const double rr = sqrt(-2.0 * log(u1));
        const double t = 6.283185307179586476925 * u2;
        buf[i] = (float)(sigma * rr * cos(t));
        if (i + 1 < k) buf[i + 1] = (float)(sigma * rr * sin(t));
    }
}

}  // namespace

extern "C" {

// n values ~ N(0, sigma), f32, from the stream seeded with `seed`.
void llamd_synth_normal(uint64_t seed, float sigma, float *out, size_t n) {
    SplitMix64 g(seed);
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = g.unit(), u2 = g.unit();
        const double r = sqrt(-2.0 * log(u1));
        const double t = 6.283185307179586476925 * u2;
        out[i] = (float)(sigma * r * cos(t));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * sin(t));
    }
}

uint16_t llamd_synth_f32_to_f16(float f) { return f32_to_f16_rne(f); }

// x: rows*k floats (k multiple of 256) -> rows*k/256 blocks of 210 bytes.
int llamd_synth_quantize_q6k(const float *x, size_t rows, size_t k, uint8_t *out) {
    if (k % 256) return -1;
    const size_t nb = rows * (k / 256);
    for (size_t b = 0; b < nb; ++b) quantize_block_q6k(x + b * 256, out + b * 210);
    return 0;
}

int llamd_synth_quantize_q8_0(const float *x, size_t rows, size_t k, uint8_t *out) {
    if (k % 32) return -1;
    const size_t nb = rows * (k / 32);
    for (size_t b = 0; b < nb; ++b) quantize_block_q8_0(x + b * 32, out + b * 34);
    return 0;
}


// Draws N(0, sigma) weights for rows x k (row-seeded, see for_rows) and
// quantizes to Q6_K row by row, so a 151936 x 2048 LM head never needs a
// 1.2 GB f32 staging buffer.
int llamd_synth_q6k_matrix(uint64_t seed, float sigma, size_t rows, size_t k, uint8_t *out) {
    if (k % 256) return -1;
    for_rows(rows, [&](size_t r) {
        std::vector<float> buf(k);
        normal_row(seed, r, sigma, buf.data(), k);
        for (size_t b = 0; b < k / 256; ++b)
            quantize_block_q6k(buf.data() + b * 256, out + (r * (k / 256) + b) * 210);
    });
    return 0;
}

int llamd_synth_q8_0_matrix(uint64_t seed, float sigma, size_t rows, size_t k, uint8_t *out) {
    if (k % 32) return -1;
    for_rows(rows, [&](size_t r) {
        std::vector<float> buf(k);
        normal_row(seed, r, sigma, buf.data(), k);
        for (size_t b = 0; b < k / 32; ++b)
            quantize_block_q8_0(buf.data() + b * 32, out + (r * (k / 32) + b) * 34);
    });
    return 0;
}

// Prefill routing: for each of n_tok tokens, n_used DISTINCT experts drawn
// without replacement from Zipf(s) over a seeded permutation of n_expert
// experts (rank r has weight 1/(r+1)^s), and positive routing weights that
// sum to one (a softmax of N(0,1) draws, renormalised as route() does).
int llamd_synth_zipf_routing(uint64_t seed, double s, size_t n_tok, size_t n_expert,
                             size_t n_used, uint32_t *ids, float *weights) {
    if (n_used == 0 || n_used > n_expert || n_expert > 4096) return -1;
    SplitMix64 g(seed);
    std::vector<uint32_t> perm(n_expert);
    for (size_t i = 0; i < n_expert; ++i) perm[i] = (uint32_t)i;
    for (size_t i = n_expert - 1; i > 0; --i) std::swap(perm[i], perm[g.next() % (i + 1)]);
    std::vector<double> w(n_expert);
    for (size_t r = 0; r < n_expert; ++r) w[r] = 1.0 / pow((double)(r + 1), s);
    std::vector<char> used(n_expert);
    for (size_t t = 0; t < n_tok; ++t) {
        std::fill(used.begin(), used.end(), 0);
        double total = 0;
        for (size_t r = 0; r < n_expert; ++r) total += w[r];
        float raw[4096];
        float sum = 0.f;
        for (size_t k = 0; k < n_used; ++k) {
            double u = g.unit() * total, acc = 0;
            size_t pick = n_expert - 1;
            for (size_t r = 0; r < n_expert; ++r) {
                if (used[r]) continue;
                acc += w[r];
                if (u <= acc) { pick = r; break; }
            }
            while (used[pick]) pick = (pick + n_expert - 1) % n_expert;
            used[pick] = 1;
            total -= w[pick];
            ids[t * n_used + k] = perm[pick];
            const double u1 = g.unit(), u2 = g.unit();
            const float z = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
            raw[k] = expf(z);
            sum += raw[k];
        }
        for (size_t k = 0; k < n_used; ++k) weights[t * n_used + k] = raw[k] / sum;
    }
    return 0;
}

}  // extern "C"
