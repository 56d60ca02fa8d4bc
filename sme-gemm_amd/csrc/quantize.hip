// Load-time quantizers: f32 weights to the reference's public input formats
// (host code; the result is then uploaded with smg_q4_create / smg_q2_create /
// smg_q1_create, as the reference's quantize functions end in
// Q4Weights::with_params / Q2Weights::new / Q1Weights::new).
//
//   smg_q4_quantize  <- Q4Weights::quantize (src/kernels/q4/quantize.rs:29-81)
//   smg_q2_quantize  <- Q2Weights::quantize (src/kernels/lowbit/q2.rs:110-143)
//   smg_q1_quantize  <- Q1Weights::quantize (src/kernels/lowbit/q1.rs:116-147)
//
// All arithmetic is f32 in the reference's order (this file is built with
// -ffp-contract=off, so no product is fused into a sum); f16 values are
// rounded to nearest even from f32 (half::f16::from_f32).
#include <cmath>
#include <cstdint>
#include <cstring>

#include "kernels.h"

namespace {

uint16_t f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u)  // inf, or NaN kept quiet with its top payload bits
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x0200u | ((ax >> 13) & 0x3FFu) : 0u));
    const int e = (int)(ax >> 23) - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        // f16 subnormal (or zero): round(|f| * 2^24) to nearest even; 1024
        // carries into the smallest normal
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)std::nearbyint((double)a * 16777216.0));
    }
    const uint32_t mant = ax & 0x7FFFFFu, hm = mant >> 13, rem = mant & 0x1FFFu;
    const uint32_t up = rem > 0x1000u || (rem == 0x1000u && (hm & 1u));
    return (uint16_t)(sign | (((uint32_t)e << 10) + hm + up));  // a carry may reach infinity
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;  // m * 2^-24, exact
        std::memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

bool pow2(size_t b) { return b && !(b & (b - 1)); }

float at(const float *w, int layout, size_t n, size_t k, size_t j, size_t d) {
    return layout == 0 ? w[j * k + d] : w[d * n + j];  // OutIn : InOut
}

}  // namespace

extern "C" {

int smg_q4_quantize(const float *w, int layout, size_t n, size_t k, size_t block, int affine,
                    uint8_t *quants, uint16_t *scales, uint16_t *mins) {
    if (!pow2(block)) return smg::report(SMG_EINVAL, "q4 block size must be a power of two");
    if (layout != 0 && layout != 1) return smg::report(SMG_EINVAL, "unknown weight layout");
    if (n && k && (!w || !quants || !scales || (affine && !mins)))
        return smg::report(SMG_EINVAL, "null array");
    const size_t nbk = (k + block - 1) / block;
    std::memset(quants, 0, (k * n + 1) / 2);
    for (size_t j = 0; j < n; j++) {
        for (size_t b = 0; b < nbk; b++) {
            const size_t d0 = b * block, d1 = d0 + block < k ? d0 + block : k;
            uint16_t s16, m16 = 0;
            if (affine) {
                float lo = INFINITY, hi = -INFINITY;
                for (size_t d = d0; d < d1; d++) {
                    const float x = at(w, layout, n, k, j, d);
                    lo = std::fmin(lo, x);  // f32::min / f32::max: a NaN operand yields the other
                    hi = std::fmax(hi, x);
                }
                s16 = f16_rne((hi - lo) / 15.0f);  // codes -8..7 over lo..hi: min sits at code 0
                const float s8 = 8.0f * f16_to_f32(s16);
                m16 = f16_rne(lo + s8);
            } else {
                float m = 0.0f;  // the largest-magnitude value, the first of equals
                for (size_t d = d0; d < d1; d++) {
                    const float x = at(w, layout, n, k, j, d);
                    if (std::fabs(x) > std::fabs(m)) m = x;
                }
                s16 = f16_rne(m / -8.0f);
            }
            scales[j * nbk + b] = s16;
            if (affine) mins[j * nbk + b] = m16;
            const float s = f16_to_f32(s16), mm = f16_to_f32(m16);
            const float inv = s == 0.0f ? 0.0f : 1.0f / s;
            for (size_t d = d0; d < d1; d++) {
                const float v = std::round((at(w, layout, n, k, j, d) - mm) * inv);  // half away from zero
                const int code = std::isnan(v) ? 0 : (int)std::fmin(std::fmax(v, -8.0f), 7.0f);
                const size_t idx = d * n + j;
                quants[idx / 2] |= (uint8_t)(((uint32_t)code & 0x0Fu) << (4 * (idx % 2)));
            }
        }
    }
    return SMG_OK;
}

int smg_q2_quantize(const float *w, int layout, size_t n, size_t k, size_t block,
                    const int8_t *codebook, uint8_t *codes, uint16_t *scales) {
    if (!pow2(block) || block < 16 || block > 65536)
        return smg::report(SMG_EINVAL, "q2 block size must be a power of two from 16 to 65536");
    if (layout != 0 && layout != 1) return smg::report(SMG_EINVAL, "unknown weight layout");
    if (!codebook || (n && k && (!w || !codes || !scales))) return smg::report(SMG_EINVAL, "null array");
    float cb[4];
    float cmax = 0.0f;
    for (int i = 0; i < 4; i++) {
        cb[i] = (float)codebook[i];
        cmax = std::fmax(cmax, std::fabs(cb[i]));
    }
    if (!(cmax > 0.0f)) return smg::report(SMG_EINVAL, "q2 codebook is all zeros");
    const size_t nbk = (k + block - 1) / block;
    std::memset(codes, 0, (k * n + 3) / 4);
    for (size_t j = 0; j < n; j++) {
        for (size_t b = 0; b < nbk; b++) {
            const size_t d0 = b * block, d1 = d0 + block < k ? d0 + block : k;
            float amax = 0.0f;
            for (size_t d = d0; d < d1; d++) amax = std::fmax(amax, std::fabs(at(w, layout, n, k, j, d)));
            const uint16_t s16 = f16_rne(amax / cmax);
            scales[j * nbk + b] = s16;
            const float s = f16_to_f32(s16);
            for (size_t d = d0; d < d1; d++) {
                const float x = at(w, layout, n, k, j, d);
                // nearest codebook value under f32::total_cmp of the distances
                // (non-negative or NaN, so their bit patterns order them); the
                // lower code wins a tie
                uint32_t best = 0, best_key = 0;
                for (uint32_t a = 0; a < 4; a++) {
                    const float prod = s * cb[a];
                    const float dist = std::fabs(x - prod);
                    uint32_t key;
                    std::memcpy(&key, &dist, 4);
                    if (a == 0 || key < best_key) {
                        best = a;
                        best_key = key;
                    }
                }
                const size_t idx = d * n + j;
                codes[idx / 4] |= (uint8_t)(best << (2 * (idx % 4)));
            }
        }
    }
    return SMG_OK;
}

int smg_q1_quantize(const float *w, int layout, size_t n, size_t k, size_t block, uint8_t *signs,
                    uint16_t *scales) {
    if (!pow2(block) || block < 16 || block > 65536)
        return smg::report(SMG_EINVAL, "q1 block size must be a power of two from 16 to 65536");
    if (layout != 0 && layout != 1) return smg::report(SMG_EINVAL, "unknown weight layout");
    if (n && k && (!w || !signs || !scales)) return smg::report(SMG_EINVAL, "null array");
    const size_t nbk = (k + block - 1) / block;
    std::memset(signs, 0, (k * n + 7) / 8);
    for (size_t j = 0; j < n; j++) {
        for (size_t b = 0; b < nbk; b++) {
            const size_t d0 = b * block, d1 = d0 + block < k ? d0 + block : k;
            float sum = 0.0f;
            for (size_t d = d0; d < d1; d++) sum += std::fabs(at(w, layout, n, k, j, d));
            scales[j * nbk + b] = f16_rne(sum / (float)(d1 - d0));  // the block's mean magnitude
            for (size_t d = d0; d < d1; d++) {
                if (at(w, layout, n, k, j, d) >= 0.0f) {  // +scale; NaN and negatives -scale
                    const size_t idx = j * k + d;           // WeightLayout::OutIn
                    signs[idx / 8] |= (uint8_t)(1u << (idx % 8));
                }
            }
        }
    }
    return SMG_OK;
}

}  // extern "C"
