// Shared device-side pieces of the gfx950 quantized-matmul library: element
// conversions, the fused op-graph epilogue, and the device weight layouts.
//
// Numerics follow the reference crate's portable path exactly where it is
// integer or rounding work (src/kernels/lowbit/matmul.rs:354-398,
// src/exec/scalar.rs:58-140, src/epilogue/mod.rs:40-110); every file of this
// library is compiled with -ffp-contract=off so a*b+c is never fused unless
// written as fmaf / fma.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/smegemm_gpu.h"

namespace smg {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef short short8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int int4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// f16 / bf16 <-> f32. f32 -> f16 is the hardware RNE convert; bf16 is RNE on
// the top half-word, NaN quieted (the `half` crate's bf16::from_f32).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// The empty asm makes x an opaque f32 register value: without it hipcc folds
// a producing multiply or FMA into the conversion (v_fma_mixlo_f16, one
// rounding of the exact result to f16), where the reference rounds the f32
// result and then that to f16.
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
    __asm__("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}
// GatedLinear's activation on the gate (linear.rs:815-822), in f32.
__device__ __forceinline__ float glu_act(uint32_t act, float g) {
    if (act == EP_ACT_GELU) return 0.5f * g * (1.0f + tanhf(0.7978846f * (g + 0.044715f * g * g * g)));
    return g / (1.0f + expf(-g));
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}
// The hardware hands consecutive workgroups of a 1-D grid to the 8 XCDs in
// turn (each XCD has its own L2). Renumber them so each XCD owns one
// contiguous run of logical tiles: neighbouring tiles share cache lines
// (e.g. the 128-byte line of 64 columns' scales), and those lines are then
// fetched into one L2 instead of four. A bijection for any grid size.
constexpr uint32_t N_XCD = 8;
__device__ __forceinline__ uint32_t xcd_tile(uint32_t b, uint32_t grid) {
    const uint32_t base = grid / N_XCD, rem = grid % N_XCD;
    const uint32_t x = b % N_XCD, slot = b / N_XCD;
    return (x < rem ? x * (base + 1) : rem * (base + 1) + (x - rem) * base) + slot;
}

template <bool BF16>
__device__ __forceinline__ float to_f32(uint16_t h) {
    return BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}
template <bool BF16>
__device__ __forceinline__ uint16_t from_f32(float x) {
    return BF16 ? f32_to_bf16(x) : f32_to_f16(x);
}

// ---------------------------------------------------------------------------
// Bounds-checked buffer loads. A raw buffer load whose offset lies past the
// resource's byte count returns zero in hardware, so edge handling needs no
// branch (a branch around a load makes the compiler wait on every load in
// flight). Offsets are 32-bit: a resource spans < 2 GiB.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t OOB = 0x80000000u;  // an offset no resource reaches

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ uint4 bload16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Streaming forms (the nt cache policy): data read once per call, such as a
// GEMV's weights, so that it does not displace what later calls reuse.
__device__ __forceinline__ uint4 bload16_nt(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
__device__ __forceinline__ uint16_t bload2_nt(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 2);
}
__device__ __forceinline__ uint16_t bload2(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint2 bload8(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint2 bload8_nt(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2));
}

// 8 consecutive 16-bit elements A[row][d..d+8) of a row-major [rows][k] array
// at `r` (zero outside rows x k). vec: k % 8 == 0, so rows are 16-byte aligned
// and a group of 8 is either wholly inside or wholly outside.
__device__ __forceinline__ uint4 load_row8(rsrc_t r, uint32_t row, uint32_t rows, uint32_t k,
                                           uint32_t d, bool vec) {
    if (vec) return bload16(r, (row < rows && d < k) ? (row * k + d) * 2u : OOB);
    uint16_t e[8];
#pragma unroll
    for (int q = 0; q < 8; q++)
        e[q] = bload2(r, (row < rows && d + q < k) ? (row * k + d + q) * 2u : OOB);
    return make_uint4(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                      e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16));
}

// f64 -> f16 with a single RNE rounding (half::f16::from_f64): round to f32
// with round-to-odd (f32 keeps 13 more bits than f16, so the later RNE step
// cannot double-round), then the hardware f32 -> f16 RNE convert.
__device__ __forceinline__ uint16_t f64_to_f16(double x) {
    float f = (float)x;
    double back = (double)f;
    if (back != x && x == x) {
        uint32_t u = __float_as_uint(f);
        if (fabs(back) > fabs(x)) u -= 1u;  // step toward zero (same sign)
        u |= 1u;
        f = __uint_as_float(u);
    }
    return f32_to_f16(f);
}

// ---------------------------------------------------------------------------
// Epilogue (src/exec/scalar.rs:58-140). The node list travels by value in the
// kernel arguments; operand pointers are device pointers to T (f16/bf16).
// A kernel's store applies graphs of up to EP_FUSED nodes itself (its LDS
// holds that many ROW / COL operand vectors); a longer graph, up to
// SMG_MAX_EP_NODES, is applied by ep_tail, a pass over C after a store with
// no graph -- the reference's own order, the GEMM rounded to T and then
// apply_ep_scalar over C (src/exec/macros.rs:188-206), so the results are the
// same.
// ---------------------------------------------------------------------------
constexpr int EP_FUSED = SMG_FUSED_EP_NODES;
struct EpArgs {
    uint32_t n_nodes;
    uint32_t pad;
    EpNode nodes[EP_FUSED];
    // ep_family(nodes[i].op) / ep_class(nodes[i].op), filled on the host; 32-bit
    // words so that a node index held in a scalar register reads them with a
    // scalar load (a byte at a run-time offset takes a vector load and a wait
    // for every load in flight, per node)
    uint32_t fam[EP_FUSED];
    uint32_t cls[EP_FUSED];
};
// A graph of EP_FUSED + 1 .. SMG_MAX_EP_NODES nodes, for ep_tail (2.6 KB of
// kernel arguments).
struct EpLong {
    uint32_t n_nodes;
    uint32_t pad;
    EpNode nodes[SMG_MAX_EP_NODES];
    uint32_t fam[SMG_MAX_EP_NODES];
    uint32_t cls[SMG_MAX_EP_NODES];
};

// maxNum / minNum with IEEE 754-2019 maximumNumber / minimumNumber results: a
// NaN operand yields the other operand and -0 < +0 (the AArch64 FMAXNM /
// FMINNM answer; the sign of a zero max is otherwise unspecified by Rust).
__device__ __forceinline__ double maxnumd(double x, double y) {
    if (x != x) return y;
    if (y != y) return x;
    if (x == 0.0 && y == 0.0) return (signbit(x) && signbit(y)) ? -0.0 : 0.0;
    return x > y ? x : y;
}
__device__ __forceinline__ float maxnumf(float x, float y) {
    if (x != x) return y;
    if (y != y) return x;
    if (x == 0.0f && y == 0.0f) return (signbit(x) && signbit(y)) ? -0.0f : 0.0f;
    return x > y ? x : y;
}
__device__ __forceinline__ float minnumf(float x, float y) {
    if (x != x) return y;
    if (y != y) return x;
    if (x == 0.0f && y == 0.0f) return (signbit(x) || signbit(y)) ? -0.0f : 0.0f;
    return x < y ? x : y;
}

__device__ __forceinline__ double clampd(double x, double lo, double hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

// act_apply_f64_a (src/epilogue/mod.rs:40-84), evaluated in f64 with the
// same operation order as the Rust expressions.
__device__ __forceinline__ double act_f64_body(uint32_t kind, double x, double alpha) {
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
    case 21: return 1.0507009873554805 * (x >= 0.0 ? x : 1.6732632423543772 * expm1(x));
    case 22: return maxnumd(x, 0.0) + log1p(exp(-fabs(x)));
    case 23: return x * tanh(maxnumd(x, 0.0) + log1p(exp(-fabs(x))));
    case 24: {
        // erf via Abramowitz-Stegun 7.1.26 (src/epilogue/mod.rs:86-95)
        double xe = x * 0.70710678118654752440;
        double ax = fabs(xe);
        double t = 1.0 / (1.0 + 0.3275911 * ax);
        double poly =
            ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t +
             0.254829592) *
            t;
        double e = 1.0 - poly * exp(-ax * ax);
        double erfv = xe < 0.0 ? -e : e;
        return 0.5 * x * (1.0 + erfv);
    }
    default: return x;
    }
}

// One out-of-line copy for per-cell use (GEMV stores).
__device__ __noinline__ double act_f64(uint32_t kind, double x, double alpha) {
    return act_f64_body(kind, x, alpha);
}

__device__ __forceinline__ float act_f32(uint32_t kind, float x, float alpha) {
    // kinds whose f64 formula on an f32 input is exact, or one product that
    // the f32 operation rounds the same way, inline; the rest call the f64 body
    switch (kind) {
    case 1: return maxnumf(x, 0.0f);
    case 6: return x >= 0.0f ? x : alpha * x;
    case 10: return __builtin_fabsf(x);
    case 11: return -x;
    case 12: return x * x;
    case 13: return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
    default: return (float)act_f64(kind, (double)x, (double)alpha);
    }
}

// A trailing activation's 16-bit result, to16(f32(f64 formula)), as
// from_f32<BF16>(act_f32(...)) gives it, with a fast path for the logistic
// kinds (silu 3, sigmoid 5): y = x or 1 times 1 / (1 + 2^t), t = -x*log2(e)
// carried as t_hi + t_lo (an fma recovers the product's rounding, a second term
// the constant's), on v_exp_f32 / v_rcp_f32 (1 ulp each): y is within about 4
// f32 ulps of the f64 formula, so if y scaled by 1 -+ 2^-19 (16 ulps) rounds
// to the same 16-bit value, the f64 formula's f32 value -- inside that
// interval -- rounds to it too (rounding is monotone). Otherwise, for
// non-finite values, and once e^-x passes 2^100 (x below about -69, where the
// quotient nears f32's subnormal range: at x = -90 silu is -7.4e-38, a normal
// bf16 value, that 1 / (1 + e^-x) in f32 would flush to zero), the f64 formula
// (inline for these two kinds) decides.
template <bool BF16>
__device__ __forceinline__ uint16_t act_round16(uint32_t kind, float x, float alpha) {
    if (kind == 3 || kind == 5) {
        constexpr float L_HI = 1.44269502162933349609375f;       // log2(e) rounded to f32
        constexpr float L_LO = 1.925962991e-08f;                 // log2(e) - L_HI
        const float t_hi = -x * L_HI;
        const float t_lo = __builtin_fmaf(-x, L_HI, -t_hi) + -x * L_LO;
        const float e = __builtin_amdgcn_exp2f(t_hi) * (1.0f + t_lo * 0.693147180559945309f);
        const float y = (kind == 3 ? x : 1.0f) * __builtin_amdgcn_rcpf(1.0f + e);
        if (__builtin_isfinite(x) && e < 0x1p100f && __builtin_isfinite(y)) {
            const float d = __builtin_fabsf(y) * 0x1p-19f;
            const uint16_t lo = from_f32<BF16>(y - d), hi = from_f32<BF16>(y + d);
            if (lo == hi) return lo;
        }
        // the f64 formula inline (a call would spill registers to scratch)
        const double yd = kind == 3 ? act_f64_body(3, (double)x, 0.0) : act_f64_body(5, (double)x, 0.0);
        return from_f32<BF16>((float)yd);
    }
    return from_f32<BF16>(act_f32(kind, x, alpha));
}

// The compiled store variant for an op-graph (the kernels' EPV template
// argument): 1 for no graph, 2 for [add_col] and 3 for [mul_col, add_col],
// each optionally followed by a trailing activation; 0 (the generic,
// interpreted store) for anything else. Host code.
struct EpPick {
    int v;
    const uint16_t *a, *b;
    uint32_t act;
    float alpha;
};
inline EpPick pick_ep(const EpArgs &ep) {
    EpPick p = {0, nullptr, nullptr, EP_ACT_NONE, 0.0f};
    uint32_t n = ep.n_nodes;
    if (n == 0) {
        p.v = 1;
        return p;
    }
    const EpNode &last = ep.nodes[n - 1];
    if (last.op == EP_OP_ACT) {
        p.act = last.aux;
        p.alpha = last.scalar;
        n--;
    }
    if (n == 1 && ep.nodes[0].op == EP_OP_ADD_COL) {
        p.v = 2;
        p.b = (const uint16_t *)ep.nodes[0].ptr;
    } else if (n == 2 && ep.nodes[0].op == EP_OP_MUL_COL && ep.nodes[1].op == EP_OP_ADD_COL) {
        p.v = 3;
        p.a = (const uint16_t *)ep.nodes[0].ptr;
        p.b = (const uint16_t *)ep.nodes[1].ptr;
    }
    if (p.v == 0) p = {0, nullptr, nullptr, EP_ACT_NONE, 0.0f};
    return p;
}

// Eight cells at once (GEMM stores): one call per 8 cells, the kind switch
// taken once and each case's f64 formula inlined for a constant kind.
struct F8 {
    float v[8];
};
__device__ __noinline__ F8 act8(uint32_t kind, F8 x, float alpha) {
    const double a = (double)alpha;
    switch (kind) {
#define SMG_ACT8_CASE(K)                                                                  \
    case K:                                                                               \
        _Pragma("unroll") for (int e = 0; e < 8; e++)                                     \
            x.v[e] = (float)act_f64_body(K, (double)x.v[e], a);                           \
        break;
        SMG_ACT8_CASE(1) SMG_ACT8_CASE(2) SMG_ACT8_CASE(3) SMG_ACT8_CASE(4) SMG_ACT8_CASE(5)
        SMG_ACT8_CASE(6) SMG_ACT8_CASE(7) SMG_ACT8_CASE(8) SMG_ACT8_CASE(9) SMG_ACT8_CASE(10)
        SMG_ACT8_CASE(11) SMG_ACT8_CASE(12) SMG_ACT8_CASE(13) SMG_ACT8_CASE(14)
        SMG_ACT8_CASE(15) SMG_ACT8_CASE(16) SMG_ACT8_CASE(17) SMG_ACT8_CASE(18)
        SMG_ACT8_CASE(19) SMG_ACT8_CASE(20) SMG_ACT8_CASE(21) SMG_ACT8_CASE(22)
        SMG_ACT8_CASE(23) SMG_ACT8_CASE(24)
#undef SMG_ACT8_CASE
    default:
        break;
    }
    return x;
}

// The same activations evaluated in f32 (device libm; the logistic kinds with
// the hardware 2^x and reciprocal), for the f16/bf16 GEMM
// stores, whose results are held to a tolerance rather than to the bits: the
// value then rounds to 16 bits, so it differs from the f64 formula's only when
// the two straddle a 16-bit rounding boundary (at most one 16-bit ulp).
// Piecewise-linear kinds (relu, clamps, abs, neg, sign, leaky) are exact.
__device__ __forceinline__ float clampf_(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}
// x * 1/(1 + e^-y) with the hardware 2^x and reciprocal (about 1 ulp each in
// f32): the logistic factor of silu, sigmoid and tanh-gelu. Once e^-y passes
// 2^100 the quotient is x * e^y to within 2^-100 relative, evaluated in f64:
// the f32 reciprocal of 1 + e^-y would reach the subnormal range (or zero, for
// an infinite e^-y) where the bf16 result, e.g. silu(-90) = -7.4e-38, is still
// a normal value.
__device__ __forceinline__ float mul_logistic(float x, float y) {
    const float e = __builtin_amdgcn_exp2f(-y * 1.4426950408889634f);
    if (e < 0x1p100f) return x * __builtin_amdgcn_rcpf(1.0f + e);
    return (float)((double)x * exp((double)y));
}
__device__ __forceinline__ float act_f32_fast(uint32_t kind, float x, float a) {
    switch (kind) {
    case 1: return maxnumf(x, 0.0f);
    // 0.5 x (1 + tanh(u)) = x / (1 + e^-2u)
    case 2: return mul_logistic(x, 2.0f * 0.7978845608028654f * (x + 0.044715f * x * x * x));
    case 3: return mul_logistic(x, x);
    case 4: return tanhf(x);
    case 5: return mul_logistic(1.0f, x);
    case 6: return x >= 0.0f ? x : a * x;
    case 7: return clampf_(x, 0.0f, 6.0f);
    case 8: return clampf_(x / 6.0f + 0.5f, 0.0f, 1.0f);
    case 9: return x * clampf_(x / 6.0f + 0.5f, 0.0f, 1.0f);
    case 10: return fabsf(x);
    case 11: return -x;
    case 12: return x * x;
    case 13: return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
    case 14: return sqrtf(x);
    case 15: return x / (1.0f + fabsf(x));
    case 16: return 1.0f / x;
    case 17: return 1.0f / sqrtf(x);
    case 18: return expf(x);
    case 19: return logf(x);
    case 20: return x >= 0.0f ? x : a * expm1f(x);
    case 21: return 1.0507009873554805f * (x >= 0.0f ? x : 1.6732632423543772f * expm1f(x));
    case 22: return maxnumf(x, 0.0f) + log1pf(expf(-fabsf(x)));
    case 23: return x * tanhf(maxnumf(x, 0.0f) + log1pf(expf(-fabsf(x))));
    case 24: {
        const float xe = x * 0.70710678118654752440f, ax = fabsf(xe);
        const float t = 1.0f / (1.0f + 0.3275911f * ax);
        const float poly =
            ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
        const float e = 1.0f - poly * expf(-ax * ax);
        return 0.5f * x * (1.0f + (xe < 0.0f ? -e : e));
    }
    default: return x;
    }
}
__device__ __noinline__ F8 act8_fast(uint32_t kind, F8 x, float alpha) {
    switch (kind) {
#define SMG_ACT8F_CASE(K)                                                                 \
    case K:                                                                               \
        _Pragma("unroll") for (int e = 0; e < 8; e++) x.v[e] = act_f32_fast(K, x.v[e], alpha); \
        break;
        SMG_ACT8F_CASE(1) SMG_ACT8F_CASE(2) SMG_ACT8F_CASE(3) SMG_ACT8F_CASE(4) SMG_ACT8F_CASE(5)
        SMG_ACT8F_CASE(6) SMG_ACT8F_CASE(7) SMG_ACT8F_CASE(8) SMG_ACT8F_CASE(9) SMG_ACT8F_CASE(10)
        SMG_ACT8F_CASE(11) SMG_ACT8F_CASE(12) SMG_ACT8F_CASE(13) SMG_ACT8F_CASE(14)
        SMG_ACT8F_CASE(15) SMG_ACT8F_CASE(16) SMG_ACT8F_CASE(17) SMG_ACT8F_CASE(18)
        SMG_ACT8F_CASE(19) SMG_ACT8F_CASE(20) SMG_ACT8F_CASE(21) SMG_ACT8F_CASE(22)
        SMG_ACT8F_CASE(23) SMG_ACT8F_CASE(24)
#undef SMG_ACT8F_CASE
    default:
        break;
    }
    return x;
}

// Operand class of an op-graph node: which operand element a cell reads.
enum EpClass : uint32_t { EPC_SCALAR = 0, EPC_ROW = 1, EPC_COL = 2, EPC_TENSOR = 3 };
// Arithmetic family of a node.
enum EpFamily : uint32_t { EPF_ADD = 0, EPF_MUL, EPF_SUB, EPF_DIV, EPF_MAX, EPF_MIN, EPF_ACT, EPF_NONE };

__host__ __device__ constexpr uint32_t ep_class(uint32_t op) {
    switch (op) {
    case EP_OP_ADD_ROW: case EP_OP_MUL_ROW: case EP_OP_SUB_ROW: case EP_OP_DIV_ROW:
    case EP_OP_MAX_ROW: case EP_OP_MIN_ROW:
        return EPC_ROW;
    case EP_OP_ADD_COL: case EP_OP_MUL_COL: case EP_OP_SUB_COL: case EP_OP_DIV_COL:
    case EP_OP_MAX_COL: case EP_OP_MIN_COL:
        return EPC_COL;
    case EP_OP_ADD_TENSOR: case EP_OP_MUL_TENSOR: case EP_OP_SUB_TENSOR:
    case EP_OP_DIV_TENSOR: case EP_OP_MAX_TENSOR: case EP_OP_MIN_TENSOR:
        return EPC_TENSOR;
    default:
        return EPC_SCALAR;  // scalar ops read nd.scalar; ACT reads nothing
    }
}

__host__ __device__ constexpr uint32_t ep_family(uint32_t op) {
    switch (op) {
    case EP_OP_ADD_SCALAR: case EP_OP_ADD_ROW: case EP_OP_ADD_COL: case EP_OP_ADD_TENSOR:
        return EPF_ADD;
    case EP_OP_MUL_SCALAR: case EP_OP_MUL_ROW: case EP_OP_MUL_COL: case EP_OP_MUL_TENSOR:
        return EPF_MUL;
    case EP_OP_SUB_SCALAR: case EP_OP_SUB_ROW: case EP_OP_SUB_COL: case EP_OP_SUB_TENSOR:
        return EPF_SUB;
    case EP_OP_DIV_SCALAR: case EP_OP_DIV_ROW: case EP_OP_DIV_COL: case EP_OP_DIV_TENSOR:
        return EPF_DIV;
    case EP_OP_MAX_SCALAR: case EP_OP_MAX_ROW: case EP_OP_MAX_COL: case EP_OP_MAX_TENSOR:
        return EPF_MAX;
    case EP_OP_MIN_SCALAR: case EP_OP_MIN_ROW: case EP_OP_MIN_COL: case EP_OP_MIN_TENSOR:
        return EPF_MIN;
    case EP_OP_ACT:
        return EPF_ACT;
    default:
        return EPF_NONE;
    }
}

// One non-activation node applied to one value; v is the node's operand (f32
// of the T element, or the scalar) (src/exec/scalar.rs:28-53).
__device__ __forceinline__ float ep_arith(uint32_t fam, float x, float v) {
    switch (fam) {
    case EPF_ADD: return x + v;
    case EPF_MUL: return x * v;
    case EPF_SUB: return x - v;
    case EPF_DIV: return __fdiv_rn(x, v);
    case EPF_MAX: return maxnumf(x, v);
    case EPF_MIN: return minnumf(x, v);
    default: return x;
    }
}

// One cell of the op-graph: x is the f32 value of the already-rounded GEMM
// output; (i, j) its row and column; n the row length used when a TENSOR
// node's ld is 0. Nodes apply in order (the trailing activation is the last
// node, as resolve_nodes appends it: src/exec/scalar.rs:28-53).
template <bool BF16, class E>
__device__ uint16_t ep_cell(const E &ep, float x, size_t i, size_t j, size_t n) {
    for (uint32_t t = 0; t < ep.n_nodes; t++) {
        const EpNode &nd = ep.nodes[t];
        const uint16_t *p = (const uint16_t *)nd.ptr;
        float v = nd.scalar;
        switch (ep.cls[t]) {
        case EPC_ROW: v = to_f32<BF16>(p[i]); break;
        case EPC_COL: v = to_f32<BF16>(p[j]); break;
        case EPC_TENSOR: v = to_f32<BF16>(p[i * (nd.ld == 0 ? n : nd.ld) + j]); break;
        default: break;
        }
        if (ep.fam[t] == EPF_ACT && t + 1 == ep.n_nodes) return act_round16<BF16>(nd.aux, x, nd.scalar);
        x = ep.fam[t] == EPF_ACT ? act_f32(nd.aux, x, nd.scalar) : ep_arith(ep.fam[t], x, v);
    }
    return from_f32<BF16>(x);
}

// Operands of the first EP_PRE nodes of one cell, loaded ahead of time (raw
// 16-bit elements; scalar nodes need none) so a kernel can issue these loads
// with its other early loads instead of after its result is ready.
constexpr int EP_PRE = 4;
struct EpPre {
    uint32_t raw[EP_PRE];
};
__device__ __forceinline__ EpPre ep_prefetch(const EpArgs &ep, size_t i, size_t j, size_t n) {
    EpPre pre;
#pragma unroll
    for (int q = 0; q < EP_PRE; q++) {
        pre.raw[q] = 0;
        if ((uint32_t)q < ep.n_nodes) {
            const EpNode &nd = ep.nodes[q];
            const uint16_t *p = (const uint16_t *)nd.ptr;
            switch (ep.cls[q]) {
            case EPC_ROW: pre.raw[q] = p[i]; break;
            case EPC_COL: pre.raw[q] = p[j]; break;
            case EPC_TENSOR: pre.raw[q] = p[i * (nd.ld == 0 ? n : nd.ld) + j]; break;
            default: break;
            }
        }
    }
    return pre;
}

// finish() with the first EP_PRE operands taken from ep_prefetch.
template <bool BF16>
__device__ __forceinline__ uint16_t finish_pre(const EpArgs &ep, EpPre pre, float acc, size_t i,
                                               size_t j, size_t n) {
    // the prefetched elements are first read here: without this the compiler
    // may convert them right after their loads, waiting there for every load
    // issued before them
#pragma unroll
    for (int q = 0; q < EP_PRE; q++) asm volatile("" : "+v"(pre.raw[q]));
    uint16_t c = from_f32<BF16>(acc);
    if (ep.n_nodes == 0) return c;
    float x = to_f32<BF16>(c);
#pragma unroll
    for (int q = 0; q < EP_PRE; q++) {
        if ((uint32_t)q < ep.n_nodes) {
            const EpNode &nd = ep.nodes[q];
            const float v = ep.cls[q] == EPC_SCALAR ? nd.scalar : to_f32<BF16>((uint16_t)pre.raw[q]);
            if (ep.fam[q] == EPF_ACT && (uint32_t)q + 1 == ep.n_nodes) return act_round16<BF16>(nd.aux, x, nd.scalar);
            x = ep.fam[q] == EPF_ACT ? act_f32(nd.aux, x, nd.scalar) : ep_arith(ep.fam[q], x, v);
        }
    }
    for (uint32_t q = EP_PRE; q < ep.n_nodes; q++) {
        const EpNode &nd = ep.nodes[q];
        const uint16_t *p = (const uint16_t *)nd.ptr;
        float v = nd.scalar;
        switch (ep.cls[q]) {
        case EPC_ROW: v = to_f32<BF16>(p[i]); break;
        case EPC_COL: v = to_f32<BF16>(p[j]); break;
        case EPC_TENSOR: v = to_f32<BF16>(p[i * (nd.ld == 0 ? n : nd.ld) + j]); break;
        default: break;
        }
        if (ep.fam[q] == EPF_ACT && q + 1 == ep.n_nodes) return act_round16<BF16>(nd.aux, x, nd.scalar);
        x = ep.fam[q] == EPF_ACT ? act_f32(nd.aux, x, nd.scalar) : ep_arith(ep.fam[q], x, v);
    }
    return from_f32<BF16>(x);
}

// Final store of one output: round the accumulator-derived value to T, then
// (iff the graph is non-empty) run the graph in f32 on that rounded value and
// round again -- "GEMM to T, then apply_ep_scalar" (src/exec/macros.rs:188-206).
template <bool BF16>
__device__ __forceinline__ uint16_t finish(const EpArgs &ep, float acc, size_t i, size_t j,
                                           size_t n) {
    uint16_t c = from_f32<BF16>(acc);
    if (ep.n_nodes == 0) return c;
    return ep_cell<BF16>(ep, to_f32<BF16>(c), i, j, n);
}

// ---------------------------------------------------------------------------
// Device weight layouts (this library's own; the reference's band-major
// arrays are repacked into these at upload).
//
// Every array is a grid of fixed-size cells, [rows][n_pad] (a Q4 chunk, a
// low-bit lane group, a scale or a min), stored in blocks of 4 rows x 16
// columns: a block holds its 4 rows' 16 cells each, and blocks run along a
// row of blocks (one 4-row band across all columns) before the next band.
// Cell (r, j) is cell number cell_index(r, j, rows, n_pad). For Q4 a block
// is 1 KB, what one wave of the decode GEMV loads in one step (4 chunks of
// its 16 columns), and the workgroups on neighbouring column tiles read
// neighbouring blocks, so the grid as a whole streams through memory in
// order. (Measured against a row-major grid, where a wave's step reads four
// 256-byte pieces, and against whole-column tiles, where each workgroup
// reads its own distant region: the single-row GEMV from HBM takes 4.55 us
// here against 4.9 and 5.2.) Allocations round rows up to whole blocks.
//
// Q4: K is cut into chunks of 32 depths (16 bytes); chunk kc of column j is
// cell (kc, j) of a grid of nchunks rows. Inside a chunk, dword w
// (depths 8w..8w+7) holds depth 8w+2e at bits 4e..4e+3 and depth 8w+2e+1 at
// bits 16+4e..16+4e+3 (e = 0..3), so ((dword >> 4e) & 0x000F000F) yields the
// consecutive pair (8w+2e, 8w+2e+1) in two half-words. The stored nibble is
// code + 8 (0..15): the reference's two's-complement nibble
// (q4/mod.rs:205-214) with its top bit flipped at upload, so the dequant
// subtracts a constant instead of sign-extending.
// Scales (and mins): cell (kb = d/block, j) of an f16 grid of sc_rows rows.
//
// Low-bit (Q2 / Q1) layouts are cut for v_mfma_i32_16x16x64_i8, whose A
// operand gives each lane 16 depths of one column: K is split into 64-depth
// slabs, a slab into four 16-depth quarters g. A "group" is the 16 bytes one
// lane loads: quarter g of several consecutive slabs of one column. The four
// quarters of group q of column j make the 64-byte cell (q, j) (quarter g at
// byte 16g), so 16 columns of one group are 1 KB.
// Q2: a group covers 4 slabs (256 depths); dword u is slab 4q+u, quarter g,
//   depth 16g+4i+b of the slab at byte b, bits 2i..2i+1, so
//   ((dword >> 2i) & 0x03030303) gives 4 consecutive depths' codes as bytes.
// Q1: a group covers 8 slabs (512 depths); dword u holds slabs 8q+2u (bit i of
//   byte b = depth 16g+4i+b, i < 4) and 8q+2u+1 (bit 4+i of byte b), so
//   ((dword >> i) & 0x01010101) gives 4 consecutive sign bits as 0/1 bytes.
// Low-bit scales: cell (block, j) of an f16 grid of sc_rows rows.
// ---------------------------------------------------------------------------
constexpr int Q4_CHUNK = 32;    // depths per 16-byte Q4 chunk
constexpr int LB_SLAB = 64;     // depths per MFMA K step
constexpr int Q2_GROUP = 256;   // depths per 16-byte Q2 lane group
constexpr int Q1_GROUP = 512;   // depths per 16-byte Q1 lane group

// Byte offset of the dword holding (depth d, column j) in a low-bit layout,
// and the bit of depth d inside that dword.
// Cell number of cell (r, j) of a grid of `rows` rows and n_pad columns: a
// part from the row plus a part from the column (so a DMA can take the row's
// part as its scalar base and the column's as each lane's offset).
__host__ __device__ __forceinline__ size_t cell_row_part(size_t r, size_t rows, size_t n_pad) {
    (void)rows;
    return (r >> 2) * (n_pad << 2) + (r & 3) * 16;
}
__host__ __device__ __forceinline__ size_t cell_col_part(size_t j, size_t rows, size_t n_pad) {
    (void)rows;
    (void)n_pad;
    return (j >> 4) * 64 + (j & 15);
}
__host__ __device__ __forceinline__ size_t cell_index(size_t r, size_t j, size_t rows, size_t n_pad) {
    return cell_row_part(r, rows, n_pad) + cell_col_part(j, rows, n_pad);
}
// Rows a grid of `rows` rows is allocated with: whole 4-row blocks.
__host__ __device__ __forceinline__ size_t cell_grid_rows(size_t rows) { return (rows + 3) / 4 * 4; }

template <int KIND>
__host__ __device__ __forceinline__ size_t lb_dword_offset(size_t d, size_t j, size_t ngroups, size_t n_pad) {
    const size_t grp = KIND == 2 ? Q2_GROUP : Q1_GROUP;
    const size_t q = d / grp, slab = (d % grp) / LB_SLAB, g = (d % LB_SLAB) / 16;
    const size_t u = KIND == 2 ? slab : slab / 2;
    return (cell_index(q, j, ngroups, n_pad) * 4 + g) * 16 + u * 4;
}
template <int KIND>
__host__ __device__ __forceinline__ uint32_t lb_bit(size_t d) {
    const uint32_t x = (uint32_t)(d % 16), i = x / 4, b = x % 4;
    if (KIND == 2) return 8 * b + 2 * i;
    const uint32_t h = (uint32_t)((d % Q1_GROUP) / LB_SLAB) % 2;
    return 8 * b + 4 * h + i;
}

// ---- Q4 dequant in registers -------------------------------------------------

// v_bfi_b32 (mask in an SGPR, both data operands in VGPRs): the compiler
// otherwise splits the insert into an and + an or with literal constants.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t x, uint32_t y) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(x), "v"(y));
    return r;
}

// dword of 8 biased nibbles (code+8; depth 2e at bits 4e, depth 2e+1 at bits
// 16+4e) -> 8 f16 weights f16_RNE(scale*code) in depth order.
__device__ __forceinline__ uint4 q4_deq8(uint32_t q, half2_t s2, uint32_t mag_lo, uint32_t mag_hi) {
    const half2_t off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};  // 0x6400|u = 1024+u
    const half2_t off_hi = {(_Float16)72.0f, (_Float16)72.0f};      // 0x5400|u<<4 = 64+u
    const uint32_t q8 = q >> 8;
    // one v_bfi_b32 each: (mask & x) | (~mask & magic)
    const uint32_t h0 = bfi(0x000F000Fu, q, mag_lo);
    const uint32_t h1 = bfi(0x00F000F0u, q, mag_hi);
    const uint32_t h2 = bfi(0x000F000Fu, q8, mag_lo);
    const uint32_t h3 = bfi(0x00F000F0u, q8, mag_hi);
    const half2_t w0 = (__builtin_bit_cast(half2_t, h0) - off_lo) * s2;
    const half2_t w1 = (__builtin_bit_cast(half2_t, h1) - off_hi) * s2;
    const half2_t w2 = (__builtin_bit_cast(half2_t, h2) - off_lo) * s2;
    const half2_t w3 = (__builtin_bit_cast(half2_t, h3) - off_hi) * s2;
    return make_uint4(__builtin_bit_cast(uint32_t, w0), __builtin_bit_cast(uint32_t, w1),
                      __builtin_bit_cast(uint32_t, w2), __builtin_bit_cast(uint32_t, w3));
}


// Q4_1: 8 f16 weights f16_RNE(scale*code + min) -- one v_pk_fma_f16 per pair
// rounds the exact value once, as the reference's f16::from_f64 of the f64 sum.
__device__ __forceinline__ uint4 q4_deq8_affine(uint32_t q, half2_t s2, half2_t m2, uint32_t mag_lo,
                                                uint32_t mag_hi) {
    const half2_t off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t off_hi = {(_Float16)72.0f, (_Float16)72.0f};
    const uint32_t q8 = q >> 8;
    const half2_t c0 = __builtin_bit_cast(half2_t, bfi(0x000F000Fu, q, mag_lo)) - off_lo;
    const half2_t c1 = __builtin_bit_cast(half2_t, bfi(0x00F000F0u, q, mag_hi)) - off_hi;
    const half2_t c2 = __builtin_bit_cast(half2_t, bfi(0x000F000Fu, q8, mag_lo)) - off_lo;
    const half2_t c3 = __builtin_bit_cast(half2_t, bfi(0x00F000F0u, q8, mag_hi)) - off_hi;
    return make_uint4(__builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c0, s2, m2)),
                      __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c1, s2, m2)),
                      __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c2, s2, m2)),
                      __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c3, s2, m2)));
}

// bf16 weights bf16_RNE(f32(scale) * code [+ f32(min)]), as dequant_q4_bf16
// rounds them (through f32, src/kernels/q4/weights.rs:198-201): the codes
// come out of the same bfi step as f16 values (exact small integers), and
// v_fma_mix_f32 multiplies each by the f16 scale in f32 -- the product has at
// most 15 significant bits, so it is exact -- adding mf (f32(min), or -0 so
// that a zero keeps the product's sign) with the one rounding of the f32 sum;
// v_cvt_pk_bf16_f32 then rounds pairs to bf16 (RNE).
__device__ __forceinline__ float fma_mix_lo(uint32_t c2, uint32_t s1, float add) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(c2), "v"(s1), "v"(add));
    return r;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t c2, uint32_t s1, float add) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(c2), "v"(s1), "v"(add));
    return r;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float float2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const float2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint4 q4_deq8_bf16(uint32_t q, uint32_t s1, float mf, uint32_t mag_lo, uint32_t mag_hi) {
    const half2_t off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
    const half2_t off_hi = {(_Float16)72.0f, (_Float16)72.0f};
    const uint32_t q8 = q >> 8;
    const uint32_t c[4] = {
        __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, bfi(0x000F000Fu, q, mag_lo)) - off_lo),
        __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, bfi(0x00F000F0u, q, mag_hi)) - off_hi),
        __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, bfi(0x000F000Fu, q8, mag_lo)) - off_lo),
        __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, bfi(0x00F000F0u, q8, mag_hi)) - off_hi)};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = pack_bf16x2(fma_mix_lo(c[i], s1, mf), fma_mix_hi(c[i], s1, mf));
    return make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace smg
