/*
 * CPU oracle for the quantized-weight matmul path of electricapp/sme-gemm.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C, the reference
 * crate's portable (non-SME) Rust path, which is what every entry point runs
 * off Apple silicon. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker. The product path
 * (sme-gemm_amd/) never links or calls it.
 *
 * Build: `make -C oracle` (gcc, -ffp-contract=off: the Rust reference never
 * contracts a*b+c into an fma unless it writes mul_add).
 *
 * Pinning (how each part is checked against something other than itself):
 *   - f16/bf16 conversions: exhaustive / sampled comparison against numpy's
 *     float16 (direct f32->f16 and f64->f16 RNE) and torch's bfloat16 RNE
 *     (tests/test_oracle_pins.py).
 *   - Q4 dequant: closed form over every nibble x a sweep of scales, and the
 *     reference's own round-trip invariants (weights.rs:315,359,426).
 *   - gemm_f16/bf16: brute force against an independent numpy f32 sequential
 *     accumulation, plus closed forms (all-ones A -> column sums, k=0 -> 0).
 *   - epilogue: per-op closed forms against numpy/math in f64.
 *   - lowbit quantize_row/reference: numpy restatement on small shapes, the
 *     f64 activation-rounding bound of tests/correctness/q2.rs:39-77, grid
 *     recovery (q2.rs:228, q1.rs:279), and independence from m.
 *   - the decode block's passes: see tests/test_oracle_block_pins.py.
 *   - the threaded CPU baseline: bit for bit the single-threaded functions.
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 conversions (the `half` 2.7.1 crate semantics).  */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static inline uint64_t f64_bits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }

/* half::f16::to_f32 -- exact widening. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) {
        /* inf / NaN: payload moves to the top of the f32 mantissa */
        return bits_f32(sign | 0x7f800000u | (man << 13));
    }
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: value = man * 2^-24, exact in f32 */
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* Round a finite positive value given as an unbounded binary fraction
 * (mantissa m with implicit exponent e: value = m * 2^e, m < 2^63) to f16
 * bits with round-to-nearest-even. Shared by the f32 and f64 paths so both
 * are a single rounding from the exact input. */
static uint16_t round_to_f16(uint64_t m, int e) {
    /* normalise m to have its top bit at position 62 */
    if (m == 0) return 0;
    int top = 63 - __builtin_clzll(m);
    /* value = m * 2^e, leading bit weight 2^(top+e) */
    int lead = top + e; /* unbiased exponent of the value */
    if (lead > 15) return 0x7c00; /* overflow -> inf (RNE rounds >= 65520 up too) */
    /* target quantum: normals have 10 fraction bits -> quantum 2^(lead-10);
     * subnormals have fixed quantum 2^-24 */
    int q = lead - 10;
    if (q < -24) q = -24;
    /* number of bits of m below the quantum */
    int shift = q - e;
    uint64_t r;
    if (shift <= 0) {
        r = m << (-shift); /* exact */
    } else if (shift >= 64) {
        r = 0; /* value < 2^-25 * ... -> rounds to 0 unless above half quantum */
        /* value < quantum/2 ? m*2^e < 2^(q-1) holds when shift >= 64 since m < 2^63 */
    } else {
        uint64_t rem = m & ((1ull << shift) - 1);
        uint64_t half = 1ull << (shift - 1);
        r = m >> shift;
        if (rem > half || (rem == half && (r & 1))) r++;
    }
    /* r is the count of quanta; rebuild the f16 */
    if (q == -24) {
        /* subnormal range (or rounded up into the first normal binade) */
        return (uint16_t)r; /* r <= 0x400 -> 0x400 is the smallest normal: bits match */
    }
    /* normal: r in [2^10, 2^11] */
    int biased = q + 10 + 15;
    if (r == (1ull << 11)) { r >>= 1; biased++; }
    if (biased >= 31) return 0x7c00;
    return (uint16_t)((biased << 10) | (r & 0x3ff));
}

/* half::f16::from_f32 -- RNE; NaN keeps its top payload bits and is quieted. */
uint16_t or_f32_to_f16(float x) {
    uint32_t u = f32_bits(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xff;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return sign | 0x7c00;
        return sign | 0x7e00 | (uint16_t)(man >> 13);
    }
    uint64_t m;
    int e;
    if (exp == 0) { m = man; e = -149; }
    else { m = man | 0x800000u; e = (int)exp - 150; }
    return sign | round_to_f16(m, e);
}

/* half::f16::from_f64 -- one direct RNE rounding (not via f32). */
uint16_t or_f64_to_f16(double x) {
    uint64_t u = f64_bits(x);
    uint16_t sign = (uint16_t)((u >> 48) & 0x8000u);
    uint32_t exp = (uint32_t)((u >> 52) & 0x7ff);
    uint64_t man = u & 0xfffffffffffffull;
    if (exp == 0x7ff) {
        if (man == 0) return sign | 0x7c00;
        return sign | 0x7e00 | (uint16_t)(man >> 42);
    }
    uint64_t m;
    int e;
    if (exp == 0) { m = man; e = -1074; }
    else { m = man | (1ull << 52); e = (int)exp - 1075; }
    return sign | round_to_f16(m, e);
}

/* half::bf16::to_f32 -- exact. */
float or_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* half::bf16::from_f32 -- RNE on the top 16 bits; NaN quieted. */
uint16_t or_f32_to_bf16(float x) {
    uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t round_bit = 0x8000u;
    if ((u & round_bit) != 0 && (u & (3u * round_bit - 1)) != 0)
        return (uint16_t)((u >> 16) + 1);
    return (uint16_t)(u >> 16);
}

/* Rust `f64 as f32`: RNE. C's (float) cast on x86-64 SSE is RNE. */
static inline float f64_to_f32(double x) { return (float)x; }

/* ------------------------------------------------------------------------ */
/* Q4 row-major dequant: src/kernels/q4/mod.rs:193-224 (q4_rowmajor),        */
/* weights.rs:232-259 (dequant_rows). w = f64(scale)*code (+ f64(min)),      */
/* exact in f64, rounded once.                                               */
/* ------------------------------------------------------------------------ */

static inline int q4_code(const uint8_t *quants, size_t idx) {
    uint8_t byte = quants[idx / 2];
    int nib = (idx % 2 == 0) ? (byte & 0x0f) : (byte >> 4);
    return nib - (nib < 8 ? 0 : 16); /* mod.rs:213-214 two's complement */
}

/* out: k x n row-major f16 bits. mins may be NULL (Q4Form::Scale). */
void or_q4_dequant_f16(const uint8_t *quants, const uint16_t *scales, const uint16_t *mins,
                       size_t n, size_t k, size_t block, uint16_t *out) {
    size_t nbk = (k + block - 1) / block;
    for (size_t d = 0; d < k; d++) {
        for (size_t j = 0; j < n; j++) {
            size_t idx = d * n + j;
            size_t bi = j * nbk + d / block;
            double w = (double)or_f16_to_f32(scales[bi]) * (double)q4_code(quants, idx);
            if (mins) w += (double)or_f16_to_f32(mins[bi]);
            out[idx] = or_f64_to_f16(w);
        }
    }
}

/* bf16 twin: mod.rs:250-256 / weights.rs:198-201 -- `bf16::from_f32(w as f32)`,
 * i.e. f64 -> f32 (RNE) -> bf16 (RNE). */
void or_q4_dequant_bf16(const uint8_t *quants, const uint16_t *scales, const uint16_t *mins,
                        size_t n, size_t k, size_t block, uint16_t *out) {
    size_t nbk = (k + block - 1) / block;
    for (size_t d = 0; d < k; d++) {
        for (size_t j = 0; j < n; j++) {
            size_t idx = d * n + j;
            size_t bi = j * nbk + d / block;
            double w = (double)or_f16_to_f32(scales[bi]) * (double)q4_code(quants, idx);
            if (mins) w += (double)or_f16_to_f32(mins[bi]);
            out[idx] = or_f32_to_bf16(f64_to_f32(w));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Dense half-precision reference GEMM: src/reference.rs:349-387 (f16) and   */
/* :308-346 (bf16). ikj, f32 accumulator per row, K order, no contraction    */
/* (each f16 x f16 / bf16 x bf16 product is exact in f32). Output            */
/* c = to16(0 + beta*acc) (alpha = 0 as src/exec/macros.rs:188-203 passes).  */
/* col_major selects C[i,j] at c[i + j*m] (Gemm::col_major_output).          */
/* ------------------------------------------------------------------------ */

/* gemm_f16 / gemm_bf16 (src/reference.rs:308-387): C = alpha*C + beta*(A@B),
 * C[i,j] = c[i*c_rs + j*c_cs], A[i,l] = a[i*a_rs + l*a_cs], B[l,j] =
 * b[l*b_rs + j*b_cs]; ikj order with one f32 accumulator per column, then
 * prev = alpha == 0 ? 0 : alpha * C (C unread), C = T(prev + beta * acc).
 * acc: scratch of n floats. */
void or_gemm_strided(int is_bf16, size_t m, size_t n, size_t k, uint16_t *c, size_t c_rs, size_t c_cs,
                     const uint16_t *a, size_t a_rs, size_t a_cs, const uint16_t *b, size_t b_rs,
                     size_t b_cs, uint16_t alpha_bits, uint16_t beta_bits, float *acc) {
    float (*to32)(uint16_t) = is_bf16 ? or_bf16_to_f32 : or_f16_to_f32;
    uint16_t (*to16)(float) = is_bf16 ? or_f32_to_bf16 : or_f32_to_f16;
    float alpha = to32(alpha_bits), beta = to32(beta_bits);
    for (size_t i = 0; i < m; i++) {
        for (size_t j = 0; j < n; j++) acc[j] = 0.0f;
        for (size_t l = 0; l < k; l++) {
            float av = to32(a[i * a_rs + l * a_cs]);
            for (size_t j = 0; j < n; j++) {
                float p = av * to32(b[l * b_rs + j * b_cs]);
                acc[j] = acc[j] + p;
            }
        }
        for (size_t j = 0; j < n; j++) {
            uint16_t *cref = c + i * c_rs + j * c_cs;
            float prev = alpha == 0.0f ? 0.0f : alpha * to32(*cref);
            *cref = to16(prev + beta * acc[j]);
        }
    }
}

static void gemm16(int is_bf16, size_t m, size_t n, size_t k, uint16_t *c, const uint16_t *a,
                   const uint16_t *b, uint16_t beta_bits, int col_major, float *acc) {
    or_gemm_strided(is_bf16, m, n, k, c, col_major ? 1 : n, col_major ? m : 1, a, k, 1, b, n, 1, 0, beta_bits,
                    acc);
}

/* acc: scratch of n floats */
void or_gemm_f16(size_t m, size_t n, size_t k, uint16_t *c, const uint16_t *a, const uint16_t *b,
                 uint16_t beta_bits, int col_major, float *acc) {
    gemm16(0, m, n, k, c, a, b, beta_bits, col_major, acc);
}
void or_gemm_bf16(size_t m, size_t n, size_t k, uint16_t *c, const uint16_t *a, const uint16_t *b,
                  uint16_t beta_bits, int col_major, float *acc) {
    gemm16(1, m, n, k, c, a, b, beta_bits, col_major, acc);
}

/* ------------------------------------------------------------------------ */
/* Epilogue: src/exec/scalar.rs:58-140 (ep_apply_cell / apply_ep_scalar) and */
/* src/epilogue/mod.rs:40-110 (act_apply_f64_a, erf_approx).                 */
/* ------------------------------------------------------------------------ */

/* C mirror of the reference's EpNode (csrc/epilogue.h:214-221). */
typedef struct {
    uint32_t op;
    uint32_t aux;
    float scalar;
    const void *ptr;
    size_t ld;
} OrEpNode;

enum {
    OP_ADD_SCALAR = 0, OP_MUL_SCALAR = 1, OP_ADD_ROW = 2, OP_MUL_ROW = 3, OP_ADD_COL = 4,
    OP_MUL_COL = 5, OP_ADD_TENSOR = 6, OP_MUL_TENSOR = 7, OP_ACT = 8, OP_MAX_SCALAR = 9,
    OP_MIN_SCALAR = 10, OP_SUB_SCALAR = 11, OP_SUB_ROW = 12, OP_SUB_COL = 13,
    OP_SUB_TENSOR = 14, OP_DIV_SCALAR = 15, OP_DIV_ROW = 16, OP_DIV_COL = 17,
    OP_DIV_TENSOR = 18, OP_MAX_ROW = 19, OP_MAX_COL = 20, OP_MAX_TENSOR = 21,
    OP_MIN_ROW = 22, OP_MIN_COL = 23, OP_MIN_TENSOR = 24
};

/* erf via Abramowitz-Stegun 7.1.26 -- src/epilogue/mod.rs:86-95. */
static double erf_approx(double x) {
    double ax = fabs(x);
    double t = 1.0 / (1.0 + 0.3275911 * ax);
    double poly = ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t +
                   0.254829592) *
                  t;
    double e = 1.0 - poly * exp(-ax * ax);
    return x < 0.0 ? -e : e;
}

/* maxNum / minNum as IEEE 754-2019 maximumNumber / minimumNumber (a NaN
 * operand yields the other operand; -0 < +0). Rust's f32::max / f64::max
 * leave the sign of a zero result unspecified and glibc's fmax and LLVM's x86
 * lowering disagree on it; this is the AArch64 FMAXNM / FMINNM result, the
 * reference's native platform. */
static inline double maxnumd(double x, double y) {
    if (isnan(x)) return y;
    if (isnan(y)) return x;
    if (x == 0.0 && y == 0.0) return (signbit(x) && signbit(y)) ? -0.0 : 0.0;
    return x > y ? x : y;
}
static inline float maxnumf(float x, float y) {
    if (isnan(x)) return y;
    if (isnan(y)) return x;
    if (x == 0.0f && y == 0.0f) return (signbit(x) && signbit(y)) ? -0.0f : 0.0f;
    return x > y ? x : y;
}
static inline float minnumf(float x, float y) {
    if (isnan(x)) return y;
    if (isnan(y)) return x;
    if (x == 0.0f && y == 0.0f) return (signbit(x) || signbit(y)) ? -0.0f : 0.0f;
    return x < y ? x : y;
}

/* Rust f64::clamp: NaN stays NaN. */
static inline double clampd(double x, double lo, double hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* act_apply_f64_a -- src/epilogue/mod.rs:40-84. Operation order follows the
 * Rust expressions left to right (no re-association, no contraction). */
double or_act_f64(uint32_t kind, double x, double alpha) {
    const double SELU_ALPHA = 1.6732632423543772;
    const double SELU_LAMBDA = 1.0507009873554805;
    switch (kind) {
    case 1: return maxnumd(x, 0.0);
    case 2: {
        double inner = 0.7978845608028654 * (x + 0.044715 * x * x * x);
        return 0.5 * x * (1.0 + tanh(inner));
    }
    case 3: return x / (1.0 + exp(-x));
    case 4: return tanh(x);
    case 5: return 1.0 / (1.0 + exp(-x));
    case 6: return x >= 0.0 ? x : alpha * x;
    case 7: return clampd(x, 0.0, 6.0);
    case 8: return clampd(x / 6.0 + 0.5, 0.0, 1.0);
    case 9: return x * clampd(x / 6.0 + 0.5, 0.0, 1.0);
    case 10: return fabs(x);
    case 11: return -x;
    case 12: return x * x;
    case 13: return x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : 0.0);
    case 14: return sqrt(x);
    case 15: return x / (1.0 + fabs(x));
    case 16: return 1.0 / x;
    case 17: return 1.0 / sqrt(x);
    case 18: return exp(x);
    case 19: return log(x);
    case 20: return x >= 0.0 ? x : alpha * expm1(x);
    case 21: return SELU_LAMBDA * (x >= 0.0 ? x : SELU_ALPHA * expm1(x));
    case 22: return maxnumd(x, 0.0) + log1p(exp(-fabs(x)));
    case 23: return x * tanh(maxnumd(x, 0.0) + log1p(exp(-fabs(x))));
    case 24: return 0.5 * x * (1.0 + erf_approx(x * 0.70710678118654752440));
    default: return x;
    }
}

/* act_apply_f32_a: widen, evaluate in f64, narrow (RNE). */
float or_act_f32(uint32_t kind, float x, float alpha) {
    return f64_to_f32(or_act_f64(kind, (double)x, (double)alpha));
}

static inline int is_tensor_op(uint32_t op) {
    return op == OP_ADD_TENSOR || op == OP_MUL_TENSOR || op == OP_SUB_TENSOR ||
           op == OP_DIV_TENSOR || op == OP_MAX_TENSOR || op == OP_MIN_TENSOR;
}

/* ep_apply_cell -- src/exec/scalar.rs:58-123. `act` < 0 means no trailing
 * activation; otherwise it is applied last with alpha 0 (scalar.rs:118-121).
 * Operands are f16 or bf16 (is_bf16) and read as f32. */
float or_ep_cell(const OrEpNode *nodes, size_t n_nodes, int act, int is_bf16, float x, size_t i,
                 size_t j, size_t n) {
    float (*to32)(uint16_t) = is_bf16 ? or_bf16_to_f32 : or_f16_to_f32;
    for (size_t t = 0; t < n_nodes; t++) {
        const OrEpNode *nd = &nodes[t];
        const uint16_t *p = (const uint16_t *)nd->ptr;
        size_t ld = nd->ld == 0 ? n : nd->ld;
        float v = 0.0f;
        if (is_tensor_op(nd->op)) v = to32(p[i * ld + j]);
        switch (nd->op) {
        case OP_ADD_SCALAR: x = x + nd->scalar; break;
        case OP_MUL_SCALAR: x = x * nd->scalar; break;
        case OP_ADD_ROW: x = x + to32(p[i]); break;
        case OP_MUL_ROW: x = x * to32(p[i]); break;
        case OP_ADD_COL: x = x + to32(p[j]); break;
        case OP_MUL_COL: x = x * to32(p[j]); break;
        case OP_ADD_TENSOR: x = x + v; break;
        case OP_MUL_TENSOR: x = x * v; break;
        case OP_ACT: x = or_act_f32(nd->aux, x, nd->scalar); break;
        case OP_MAX_SCALAR: x = maxnumf(x, nd->scalar); break;
        case OP_MIN_SCALAR: x = minnumf(x, nd->scalar); break;
        case OP_SUB_SCALAR: x = x - nd->scalar; break;
        case OP_DIV_SCALAR: x = x / nd->scalar; break;
        case OP_SUB_ROW: x = x - to32(p[i]); break;
        case OP_DIV_ROW: x = x / to32(p[i]); break;
        case OP_MAX_ROW: x = maxnumf(x, to32(p[i])); break;
        case OP_MIN_ROW: x = minnumf(x, to32(p[i])); break;
        case OP_SUB_COL: x = x - to32(p[j]); break;
        case OP_DIV_COL: x = x / to32(p[j]); break;
        case OP_MAX_COL: x = maxnumf(x, to32(p[j])); break;
        case OP_MIN_COL: x = minnumf(x, to32(p[j])); break;
        case OP_SUB_TENSOR: x = x - v; break;
        case OP_DIV_TENSOR: x = x / v; break;
        case OP_MAX_TENSOR: x = maxnumf(x, v); break;
        case OP_MIN_TENSOR: x = minnumf(x, v); break;
        default: break;
        }
    }
    if (act >= 0) x = or_act_f32((uint32_t)act, x, 0.0f);
    return x;
}

/* apply_ep_scalar -- scalar.rs:125-140: c[idx] = to16(cell(to32(c[idx]))). */
void or_apply_ep(uint16_t *c, size_t m, size_t n, size_t rs, size_t cs, const OrEpNode *nodes,
                 size_t n_nodes, int act, int is_bf16) {
    float (*to32)(uint16_t) = is_bf16 ? or_bf16_to_f32 : or_f16_to_f32;
    uint16_t (*to16)(float) = is_bf16 ? or_f32_to_bf16 : or_f32_to_f16;
    for (size_t i = 0; i < m; i++) {
        for (size_t j = 0; j < n; j++) {
            size_t idx = i * rs + j * cs;
            float v = or_ep_cell(nodes, n_nodes, act, is_bf16, to32(c[idx]), i, j, n);
            c[idx] = to16(v);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Low-bit path: src/kernels/lowbit/matmul.rs:354-398.                        */
/* ------------------------------------------------------------------------ */

/* quantize_row -- matmul.rs:354-371. q: k int8, s: ceil(k/block) f32. */
void or_quantize_row(const uint16_t *a, size_t k, size_t block, int8_t *q, float *s) {
    size_t nbk = (k + block - 1) / block;
    for (size_t b = 0; b < nbk; b++) {
        size_t d0 = b * block, d1 = d0 + block < k ? d0 + block : k;
        float amax = 0.0f;
        for (size_t d = d0; d < d1; d++) {
            float x = fabsf(or_f16_to_f32(a[d]));
            if (isnan(x) || isnan(amax)) amax = NAN;
            else amax = fmaxf(amax, x);
        }
        float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        s[b] = amax / 127.0f;
        for (size_t d = d0; d < d1; d++) {
            float v = or_f16_to_f32(a[d]) * inv;
            float r = nearbyintf(v); /* round-ties-even under the default mode */
            int8_t o;
            if (isnan(r)) o = 0; /* Rust `as i8`: NaN -> 0, saturating */
            else if (r >= 127.0f) o = 127;
            else if (r <= -128.0f) o = -128;
            else o = (int8_t)r;
            q[d] = o;
        }
    }
}

/* Value lookups on the reference's public INPUT formats (the band-major
 * repack is a bijection checked separately):
 *   Q2: weight idx = d*n + j is bits 2*(idx%4) of byte idx/4 (q2.rs:43-47),
 *       value = codebook[code] (matmul.rs:157-160).
 *   Q1: weight idx (OutIn: j*k + d, InOut: d*n + j) is bit idx%8 of byte
 *       idx/8 (q1.rs:35-41), value = +1 if set else -1 (matmul.rs:161-167).
 *   scales[j*nbk + blk] (f16), read as f32. */
static inline int lowbit_value(int kind, const uint8_t *codes, const int8_t *codebook,
                               int layout_inout, size_t n, size_t k, size_t d, size_t j) {
    if (kind == 2) {
        size_t idx = d * n + j;
        int code = (codes[idx / 4] >> (2 * (idx % 4))) & 3;
        return codebook[code];
    }
    size_t idx = layout_inout ? d * n + j : j * k + d;
    return ((codes[idx / 8] >> (idx % 8)) & 1) ? 1 : -1;
}

/* reference -- matmul.rs:376-398. kind 2 (Q2) or 1 (Q1). c: m x n f16 bits.
 * scratch_q: k int8, scratch_s: nbk f32. Columns [j0, j1) only, so the
 * threaded CPU baseline can split N with identical arithmetic. */
void or_lowbit_reference_cols(int kind, const uint16_t *a, const uint8_t *codes,
                              const uint16_t *scales, const int8_t *codebook, int layout_inout,
                              size_t m, size_t n, size_t k, size_t block, uint16_t *c, size_t j0,
                              size_t j1, int8_t *scratch_q, float *scratch_s) {
    size_t nbk = (k + block - 1) / block;
    for (size_t i = 0; i < m; i++) {
        or_quantize_row(a + i * k, k, block, scratch_q, scratch_s);
        for (size_t j = j0; j < j1; j++) {
            float total = 0.0f;
            for (size_t blk = 0; blk < nbk; blk++) {
                size_t d0 = blk * block, d1 = d0 + block < k ? d0 + block : k;
                int32_t sum = 0;
                for (size_t d = d0; d < d1; d++)
                    sum += (int32_t)scratch_q[d] *
                           lowbit_value(kind, codes, codebook, layout_inout, n, k, d, j);
                float f = (float)sum; /* i32 -> f32 RNE */
                float sc = or_f16_to_f32(scales[j * nbk + blk]) * scratch_s[blk];
                total = fmaf(f, sc, total);
            }
            c[i * n + j] = or_f32_to_f16(total);
        }
    }
}

void or_lowbit_reference(int kind, const uint16_t *a, const uint8_t *codes,
                         const uint16_t *scales, const int8_t *codebook, int layout_inout,
                         size_t m, size_t n, size_t k, size_t block, uint16_t *c,
                         int8_t *scratch_q, float *scratch_s) {
    or_lowbit_reference_cols(kind, a, codes, scales, codebook, layout_inout, m, n, k, block, c, 0,
                             n, scratch_q, scratch_s);
    if (k == 0)
        for (size_t t = 0; t < m * n; t++) c[t] = 0;
}

/* Codes::dequant -- matmul.rs:178-197: the MOPA route's f16 weights,
 * f16::from_f32(scale_f32 * value) (row-major k x n). */
void or_lowbit_dequant_f16(int kind, const uint8_t *codes, const uint16_t *scales,
                           const int8_t *codebook, int layout_inout, size_t n, size_t k,
                           size_t block, uint16_t *out) {
    size_t nbk = (k + block - 1) / block;
    for (size_t d = 0; d < k; d++)
        for (size_t j = 0; j < n; j++) {
            float s = or_f16_to_f32(scales[j * nbk + d / block]);
            int v = lowbit_value(kind, codes, codebook, layout_inout, n, k, d, j);
            float w = kind == 2 ? s * (float)v : (v > 0 ? s : -s);
            out[d * n + j] = or_f32_to_f16(w);
        }
}

/* ------------------------------------------------------------------------ */
/* The reference's band-major resident packs (the layouts src/ffi.rs hands   */
/* to the kernels), so the GPU library's "upload from band-major" entry      */
/* points can be checked: q4/weights.rs:89-113, lowbit/q2.rs:12-20,53-86,     */
/* 148-161, lowbit/q1.rs:47-107,186-201.                                      */
/* ------------------------------------------------------------------------ */

size_t or_q4_band_sizes(size_t n, size_t k, size_t block, size_t *nib_len, size_t *sc_len) {
    size_t nb = (n + 127) / 128, nbk = (k + block - 1) / block;
    *nib_len = nb * k * 64;
    *sc_len = nb * nbk * 128;
    return nb;
}

void or_q4_pack_band(const uint8_t *quants, const uint16_t *scales, const uint16_t *mins,
                     size_t n, size_t k, size_t block, uint8_t *nib, uint16_t *sc, uint16_t *mn) {
    size_t nib_len, sc_len;
    or_q4_band_sizes(n, k, block, &nib_len, &sc_len);
    size_t nbk = (k + block - 1) / block;
    size_t nib_per_band = k * 64, sc_per_band = nbk * 128;
    memset(nib, 0, nib_len);
    memset(sc, 0, sc_len * 2);
    if (mn) memset(mn, 0, sc_len * 2);
    for (size_t d = 0; d < k; d++)
        for (size_t j = 0; j < n; j++) {
            size_t idx = d * n + j;
            uint8_t v = (idx % 2 == 0) ? (quants[idx / 2] & 0x0f) : (quants[idx / 2] >> 4);
            size_t b = j / 128, cc = j % 128;
            nib[b * nib_per_band + d * 64 + cc / 2] |= (uint8_t)(v << (4 * (cc % 2)));
        }
    for (size_t j = 0; j < n; j++) {
        size_t b = j / 128, cc = j % 128;
        for (size_t blk = 0; blk < nbk; blk++) {
            sc[b * sc_per_band + blk * 128 + cc] = scales[j * nbk + blk];
            if (mn && mins) mn[b * sc_per_band + blk * 128 + cc] = mins[j * nbk + blk];
        }
    }
}

static inline size_t lb_scale_index(size_t sc_per_band, size_t blk, size_t j) {
    size_t cc = j % 64;
    return (j / 64) * sc_per_band + blk * 64 + (cc / 32) * 32 + 2 * (cc % 16) + (cc % 32) / 16;
}

/* kind 2: band_bytes = pad16(k)*16; kind 1: pad16(k)*8. sc_per_band = nbk*64. */
void or_lowbit_band_sizes(int kind, size_t n, size_t k, size_t block, size_t *codes_len,
                          size_t *sc_len) {
    size_t nb = (n + 63) / 64, kp = (k + 15) / 16 * 16, nbk = (k + block - 1) / block;
    *codes_len = nb * kp * (kind == 2 ? 16 : 8);
    *sc_len = nb * nbk * 64;
}

void or_lowbit_pack_band(int kind, const uint8_t *codes, const uint16_t *scales,
                         int layout_inout, size_t n, size_t k, size_t block, uint8_t *packed,
                         uint16_t *sc) {
    size_t codes_len, sc_len;
    or_lowbit_band_sizes(kind, n, k, block, &codes_len, &sc_len);
    size_t kp = (k + 15) / 16 * 16, nbk = (k + block - 1) / block;
    size_t band_bytes = kp * (kind == 2 ? 16 : 8), sc_per_band = nbk * 64;
    memset(packed, 0, codes_len);
    memset(sc, 0, sc_len * 2);
    for (size_t d = 0; d < k; d++)
        for (size_t j = 0; j < n; j++) {
            if (kind == 2) {
                size_t idx = d * n + j;
                uint8_t code = (codes[idx / 4] >> (2 * (idx % 4))) & 3;
                packed[(j / 64) * band_bytes + (d / 4) * 64 + j % 64] |=
                    (uint8_t)(code << (2 * (d % 4)));
            } else {
                size_t idx = layout_inout ? d * n + j : j * k + d;
                if ((codes[idx / 8] >> (idx % 8)) & 1) {
                    size_t cc = j % 64;
                    size_t byte = (j / 64) * band_bytes + (d / 4) * 32 + cc / 2;
                    size_t bit = 4 * (cc % 2) + d % 4;
                    packed[byte] |= (uint8_t)(1u << bit);
                }
            }
        }
    for (size_t j = 0; j < n; j++)
        for (size_t blk = 0; blk < nbk; blk++)
            sc[lb_scale_index(sc_per_band, blk, j)] = scales[j * nbk + blk];
}

/* ------------------------------------------------------------------------ */
/* Array forms of the conversions, for the Python test harness.              */
/* ------------------------------------------------------------------------ */
void or_f32_to_f16_array(const float *x, uint16_t *y, size_t len) {
    for (size_t i = 0; i < len; i++) y[i] = or_f32_to_f16(x[i]);
}
void or_f64_to_f16_array(const double *x, uint16_t *y, size_t len) {
    for (size_t i = 0; i < len; i++) y[i] = or_f64_to_f16(x[i]);
}
void or_f16_to_f32_array(const uint16_t *x, float *y, size_t len) {
    for (size_t i = 0; i < len; i++) y[i] = or_f16_to_f32(x[i]);
}
void or_f32_to_bf16_array(const float *x, uint16_t *y, size_t len) {
    for (size_t i = 0; i < len; i++) y[i] = or_f32_to_bf16(x[i]);
}
void or_act_f32_array(uint32_t kind, const float *x, float *y, size_t len, float alpha) {
    for (size_t i = 0; i < len; i++) y[i] = or_act_f32(kind, x[i], alpha);
}

/* ------------------------------------------------------------------------- */
/* Load-time quantizers, restated from the reference's f32 code: outputs are the
 * public input formats (row-major codes, idx = d*n + j; Q1 signs OutIn,
 * idx = j*k + d), scales [j][blk]. layout 0 = OutIn w[j*k+d], 1 = InOut. */
static inline float q_at(const float *w, int layout, size_t n, size_t k, size_t j, size_t d) {
    return layout == 0 ? w[j * k + d] : w[d * n + j];
}

/* Q4Weights::quantize (src/kernels/q4/quantize.rs:29-81). */
void or_q4_quantize(const float *w, int layout, size_t n, size_t k, size_t block, int affine,
                    uint8_t *quants, uint16_t *scales, uint16_t *mins) {
    size_t nbk = (k + block - 1) / block;
    memset(quants, 0, (k * n + 1) / 2);
    for (size_t j = 0; j < n; j++)
        for (size_t b = 0; b < nbk; b++) {
            size_t d0 = b * block, d1 = (b + 1) * block < k ? (b + 1) * block : k;
            uint16_t sc, mn = 0;
            if (affine) {
                float lo = INFINITY, hi = -INFINITY;
                for (size_t d = d0; d < d1; d++) {
                    float x = q_at(w, layout, n, k, j, d);
                    lo = fminf(lo, x); /* Rust f32::min / max ignore a NaN operand */
                    hi = fmaxf(hi, x);
                }
                sc = or_f32_to_f16((hi - lo) / 15.0f);
                mn = or_f32_to_f16(lo + 8.0f * or_f16_to_f32(sc));
            } else {
                float m = 0.0f;
                for (size_t d = d0; d < d1; d++) {
                    float x = q_at(w, layout, n, k, j, d);
                    if (fabsf(x) > fabsf(m)) m = x;
                }
                sc = or_f32_to_f16(m / -8.0f);
            }
            scales[j * nbk + b] = sc;
            if (affine) mins[j * nbk + b] = mn;
            float s = or_f16_to_f32(sc), mm = or_f16_to_f32(mn);
            float inv = s == 0.0f ? 0.0f : 1.0f / s;
            for (size_t d = d0; d < d1; d++) {
                float r = roundf((q_at(w, layout, n, k, j, d) - mm) * inv);
                int code = isnan(r) ? 0 : (r < -8.0f ? -8 : (r > 7.0f ? 7 : (int)r)); /* clamp, `as i8` */
                size_t idx = d * n + j;
                quants[idx / 2] |= (uint8_t)((code & 0x0f) << (4 * (idx % 2)));
            }
        }
}

/* Q2Weights::quantize (src/kernels/lowbit/q2.rs:110-143); returns 0, or -1 for
 * an all-zero codebook (the reference's assert). */
int or_q2_quantize(const float *w, int layout, size_t n, size_t k, size_t block,
                   const int8_t *codebook, uint8_t *codes, uint16_t *scales) {
    float cb[4], cmax = 0.0f;
    for (int i = 0; i < 4; i++) {
        cb[i] = (float)codebook[i];
        cmax = fmaxf(cmax, fabsf(cb[i]));
    }
    if (!(cmax > 0.0f)) return -1;
    size_t nbk = (k + block - 1) / block;
    memset(codes, 0, (k * n + 3) / 4);
    for (size_t j = 0; j < n; j++)
        for (size_t b = 0; b < nbk; b++) {
            size_t d0 = b * block, d1 = (b + 1) * block < k ? (b + 1) * block : k;
            float amax = 0.0f;
            for (size_t d = d0; d < d1; d++) amax = fmaxf(amax, fabsf(q_at(w, layout, n, k, j, d)));
            scales[j * nbk + b] = or_f32_to_f16(amax / cmax);
            float s = or_f16_to_f32(scales[j * nbk + b]);
            for (size_t d = d0; d < d1; d++) {
                float x = q_at(w, layout, n, k, j, d);
                /* min_by over total_cmp: the first minimum wins; the distances
                 * are >= 0 or (positive) NaN, ordered by their bits */
                int best = 0;
                uint32_t bk = f32_bits(fabsf(x - s * cb[0]));
                for (int a = 1; a < 4; a++) {
                    uint32_t key = f32_bits(fabsf(x - s * cb[a]));
                    if (key < bk) { bk = key; best = a; }
                }
                size_t idx = d * n + j;
                codes[idx / 4] |= (uint8_t)(best << (2 * (idx % 4)));
            }
        }
    return 0;
}

/* Q1Weights::quantize (src/kernels/lowbit/q1.rs:116-147). */
void or_q1_quantize(const float *w, int layout, size_t n, size_t k, size_t block, uint8_t *signs,
                    uint16_t *scales) {
    size_t nbk = (k + block - 1) / block;
    memset(signs, 0, (k * n + 7) / 8);
    for (size_t j = 0; j < n; j++)
        for (size_t b = 0; b < nbk; b++) {
            size_t d0 = b * block, d1 = (b + 1) * block < k ? (b + 1) * block : k;
            float sum = 0.0f;
            for (size_t d = d0; d < d1; d++) sum += fabsf(q_at(w, layout, n, k, j, d));
            scales[j * nbk + b] = or_f32_to_f16(sum / (float)(d1 - d0));
            for (size_t d = d0; d < d1; d++)
                if (q_at(w, layout, n, k, j, d) >= 0.0f) {
                    size_t idx = j * k + d;
                    signs[idx / 8] |= (uint8_t)(1u << (idx % 8));
                }
        }
}

/* ------------------------------------------------------------------------ */
/* The decode block's row-wise passes (config 5): the portable bodies of     */
/* nn::rms_norm (src/nn.rs:22-32,127-144,159), attention_kv_f16's one_row      */
/* (src/kernels/kv_attention.rs:282-325), GatedLinear's glu                   */
/* (src/linear.rs:804-826) and the NeoX RoPE of examples/bonsai/model.rs:30-99 */
/* (no YaRN scaling: mscale 1). Rust never contracts a*b+c (this file is built */
/* with -ffp-contract=off) and its f32 exp / tanh / sin / cos / f64 powf are  */
/* the platform libm's (glibc here), as these calls are.                     */
/* ------------------------------------------------------------------------ */

/* norm_row with rms = true (nn.rs:127-144): lane_sum (nn.rs:22-32) keeps 8
 * lane accumulators over whole chunks of 8, sums the tail in order, then adds
 * the 8 lanes in order and the tail; r = 1 / sqrt(mean + eps) in f32; each
 * output is (v - 0) * r * w + 0 (mean 0, no bias), left to right. */
void or_rms_norm_row(const float *x, const float *w, size_t dim, float eps, float *out) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const size_t chunks = dim / 8;
    for (size_t c = 0; c < chunks; c++)
        for (size_t i = 0; i < 8; i++) {
            const float v = x[8 * c + i] - 0.0f;
            acc[i] = acc[i] + v * v;
        }
    float tail = -0.0f; /* an f32 iterator sum starts from -0.0 */
    for (size_t t = chunks * 8; t < dim; t++) {
        const float v = x[t] - 0.0f;
        tail = tail + v * v;
    }
    float s = -0.0f;
    for (size_t i = 0; i < 8; i++) s = s + acc[i];
    s = s + tail;
    const float r = 1.0f / sqrtf(s / (float)dim + eps);
    for (size_t i = 0; i < dim; i++) out[i] = (x[i] - 0.0f) * r * w[i] + 0.0f;
}

/* nn::rms_norm into f16 (rows of `dim`; each row's f32 result rounded by
 * to_f16, RNE). */
void or_rms_norm_f16(const float *x, const float *w, size_t rows, size_t dim, float eps,
                     uint16_t *y, float *row_scratch) {
    for (size_t r = 0; r < rows; r++) {
        or_rms_norm_row(x + r * dim, w, dim, eps, row_scratch);
        for (size_t i = 0; i < dim; i++) y[r * dim + i] = or_f32_to_f16(row_scratch[i]);
    }
}

/* norm_row with rms = false (nn.rs:133-143): mean = lane_sum(x) / dim, then
 * r = 1 / sqrt(lane_sum((v - mean)^2) / dim + eps), both sums in lane_sum's
 * order (8 lane accumulators over whole chunks of 8, the tail summed in order
 * from -0.0, the lanes added in order, then the tail); each output is
 * (v - mean) * r * w + b (b = 0 without a bias), left to right. */
static float or_lane_sum(const float *x, size_t dim, float mean, int square) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const size_t chunks = dim / 8;
    for (size_t c = 0; c < chunks; c++)
        for (size_t i = 0; i < 8; i++) {
            const float v = x[8 * c + i] - mean;
            acc[i] = acc[i] + (square ? v * v : x[8 * c + i]);
        }
    float tail = -0.0f;
    for (size_t t = chunks * 8; t < dim; t++) {
        const float v = x[t] - mean;
        tail = tail + (square ? v * v : x[t]);
    }
    float s = -0.0f;
    for (size_t i = 0; i < 8; i++) s = s + acc[i];
    return s + tail;
}
void or_layer_norm_row(const float *x, const float *w, const float *b, size_t dim, float eps, float *out) {
    const float mean = or_lane_sum(x, dim, 0.0f, 0) / (float)dim;
    const float r = 1.0f / sqrtf(or_lane_sum(x, dim, mean, 1) / (float)dim + eps);
    for (size_t i = 0; i < dim; i++) out[i] = (x[i] - mean) * r * w[i] + (b ? b[i] : 0.0f);
}

/* nn::layer_norm into f16 (rows of `dim`; each row's f32 result rounded by
 * to_f16, RNE). */
void or_layer_norm_f16(const float *x, const float *w, const float *b, size_t rows, size_t dim, float eps,
                       uint16_t *y, float *row_scratch) {
    for (size_t r = 0; r < rows; r++) {
        or_layer_norm_row(x + r * dim, w, b, dim, eps, row_scratch);
        for (size_t i = 0; i < dim; i++) y[r * dim + i] = or_f32_to_f16(row_scratch[i]);
    }
}

/* Rope::new without YaRN (model.rs:38-51): inv_freq[i] = (1 / base^(2i/dim))
 * in f64, then to f32. */
void or_rope_inv_freq(size_t dim, double base, float *inv_freq) {
    for (size_t i = 0; i < dim / 2; i++)
        inv_freq[i] = (float)(1.0 / pow(base, (double)(2 * i) / (double)dim));
}

/* Rope::angles (model.rs:77-85): (pos as f32 * f).sin_cos(), times mscale 1. */
void or_rope_angles(const float *inv_freq, size_t half, size_t pos, float *cos_out,
                    float *sin_out) {
    for (size_t i = 0; i < half; i++) {
        const float a = (float)pos * inv_freq[i];
        sin_out[i] = sinf(a) * 1.0f;
        cos_out[i] = cosf(a) * 1.0f;
    }
}

/* Rope::apply (model.rs:87-99): each 2*half-wide head's halves rotated
 * against each other: x1' = u c - v s, x2' = v c + u s. */
void or_rope_apply(float *x, size_t len, const float *cos_v, const float *sin_v, size_t half) {
    for (size_t h0 = 0; h0 + 2 * half <= len; h0 += 2 * half)
        for (size_t i = 0; i < half; i++) {
            const float u = x[h0 + i], v = x[h0 + half + i];
            x[h0 + i] = u * cos_v[i] - v * sin_v[i];
            x[h0 + half + i] = v * cos_v[i] + u * sin_v[i];
        }
}

/* one_row, the portable attention_kv_f16 (kv_attention.rs:282-325): per query
 * head h (KV head h / (heads / kv_heads)): q rounded to f16 after the scale,
 * scores as f32 sums in depth order, the running max by maxNum, exp(s - max)
 * summed in key order, values accumulated in key order, then divided by the
 * sum. scores: `len` floats of scratch. */
void or_attention_kv_f16(const float *q, const uint16_t *k, const uint16_t *v, size_t len,
                         size_t heads, size_t kv_heads, size_t hd, float scale, float *out,
                         float *scores, float *qh) {
    const size_t group = heads / kv_heads, ld = kv_heads * hd;
    for (size_t h = 0; h < heads; h++) {
        const size_t off = (h / group) * hd;
        for (size_t d = 0; d < hd; d++) qh[d] = or_f16_to_f32(or_f32_to_f16(q[h * hd + d] * scale));
        float mx = -INFINITY;
        for (size_t t = 0; t < len; t++) {
            float s = -0.0f;
            for (size_t d = 0; d < hd; d++) s = s + qh[d] * or_f16_to_f32(k[t * ld + off + d]);
            scores[t] = s;
            mx = fmaxf(mx, s);
        }
        float sum = 0.0f;
        for (size_t t = 0; t < len; t++) {
            scores[t] = expf(scores[t] - mx);
            sum = sum + scores[t];
        }
        float *oh = out + h * hd;
        for (size_t d = 0; d < hd; d++) oh[d] = 0.0f;
        for (size_t t = 0; t < len; t++)
            for (size_t d = 0; d < hd; d++) oh[d] = oh[d] + scores[t] * or_f16_to_f32(v[t * ld + off + d]);
        for (size_t d = 0; d < hd; d++) oh[d] = oh[d] / sum;
    }
}

/* glu (linear.rs:804-826): m rows of 2n interleaved outputs -- each 32-column
 * chunk (the last w < 32 wide) is w gate columns then w up columns -- to
 * y = f16(act(gate) * up), act in f32: silu g / (1 + exp(-g)), or (gelu != 0)
 * the tanh form 0.5 g (1 + tanh(0.7978846 (g + 0.044715 g g g))). */
void or_glu_f16(uint16_t *y, const uint16_t *both, size_t m, size_t n, int gelu) {
    for (size_t r = 0; r < m; r++)
        for (size_t c0 = 0; c0 < n; c0 += 32) {
            const size_t w = n - c0 < 32 ? n - c0 : 32;
            for (size_t j = 0; j < w; j++) {
                const float g = or_f16_to_f32(both[r * 2 * n + 2 * c0 + j]);
                const float u = or_f16_to_f32(both[r * 2 * n + 2 * c0 + w + j]);
                const float a = gelu ? 0.5f * g * (1.0f + tanhf(0.7978846f * (g + 0.044715f * g * g * g)))
                                     : g / (1.0f + expf(-g));
                y[r * n + c0 + j] = or_f32_to_f16(a * u);
            }
        }
}

/* ------------------------------------------------------------------------ */
/* The CPU baseline's threaded mode: the portable path's per-output          */
/* arithmetic split over column ranges on host threads (each output depends  */
/* on its own column only, so the bits are the single-threaded ones).       */
/* ------------------------------------------------------------------------ */
typedef struct {
    int kind; /* 4 = Q4 (dequant + f16 GEMM), 2 / 1 = low-bit int8 reference */
    const uint16_t *a;
    const uint8_t *codes;
    const uint16_t *scales;
    const int8_t *codebook;
    size_t m, n, k, block, j0, j1;
    uint16_t *c;
    int ok;
} OrColJob;

static void *or_col_job(void *arg) {
    OrColJob *jb = (OrColJob *)arg;
    const size_t w = jb->j1 - jb->j0, k = jb->k, n = jb->n;
    jb->ok = 0;
    if (w == 0) { jb->ok = 1; return NULL; }
    if (jb->kind == 4) {
        /* q4_f16_impl (q4/matmul.rs:91-102): these columns dequantized to a
         * k x w row-major panel (the same per-weight rounding), then the
         * reference GEMM over them */
        const size_t nbk = (k + jb->block - 1) / jb->block;
        uint16_t *b = malloc(k * w * 2);
        uint16_t *cc = malloc(jb->m * w * 2);
        float *acc = malloc(w * 4);
        if (!b || !cc || !acc) { free(b); free(cc); free(acc); return NULL; }
        for (size_t d = 0; d < k; d++)
            for (size_t j = jb->j0; j < jb->j1; j++) {
                const double v = (double)or_f16_to_f32(jb->scales[j * nbk + d / jb->block]) *
                                 (double)q4_code(jb->codes, d * n + j);
                b[d * w + (j - jb->j0)] = or_f64_to_f16(v);
            }
        gemm16(0, jb->m, w, k, cc, jb->a, b, 0x3C00, 0, acc);
        for (size_t i = 0; i < jb->m; i++) memcpy(jb->c + i * n + jb->j0, cc + i * w, w * 2);
        free(b);
        free(cc);
        free(acc);
    } else {
        int8_t *q = malloc(k ? k : 1);
        float *s = malloc(((k + jb->block - 1) / jb->block + 1) * 4);
        if (!q || !s) { free(q); free(s); return NULL; }
        or_lowbit_reference_cols(jb->kind, jb->a, jb->codes, jb->scales, jb->codebook, 0, jb->m, n, k,
                                 jb->block, jb->c, jb->j0, jb->j1, q, s);
        free(q);
        free(s);
    }
    jb->ok = 1;
    return NULL;
}

/* kind 4: matmul_q4 (scale form, row-major public arrays); kind 2 / 1:
 * matmul_q2 / matmul_q1 (Q1 OutIn) without an epilogue. 0 on success. */
int or_matmul_mt(int kind, const uint16_t *a, const uint8_t *codes, const uint16_t *scales,
                 const int8_t *codebook, size_t m, size_t n, size_t k, size_t block, uint16_t *c,
                 int threads) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > n) threads = (int)(n ? n : 1);
    OrColJob *jobs = calloc((size_t)threads, sizeof(OrColJob));
    pthread_t *tid = calloc((size_t)threads, sizeof(pthread_t));
    if (!jobs || !tid) { free(jobs); free(tid); return -1; }
    for (int t = 0; t < threads; t++) {
        OrColJob jb = {kind, a, codes, scales, codebook, m, n, k, block, n * (size_t)t / (size_t)threads,
                       n * (size_t)(t + 1) / (size_t)threads, c, 0};
        jobs[t] = jb;
    }
    int rc = 0;
    char *started = calloc((size_t)threads, 1);
    if (!started) { free(jobs); free(tid); return -1; }
    for (int t = 1; t < threads; t++) {
        if (pthread_create(&tid[t], NULL, or_col_job, &jobs[t]) == 0) started[t] = 1;
        else rc = -1;
    }
    or_col_job(&jobs[0]);
    for (int t = 1; t < threads; t++)  /* every thread that started, before jobs is freed */
        if (started[t]) pthread_join(tid[t], NULL);
    free(started);
    for (int t = 0; t < threads; t++)
        if (!jobs[t].ok) rc = -1;
    free(jobs);
    free(tid);
    return rc;
}
