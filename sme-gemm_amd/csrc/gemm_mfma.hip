// Prefill-shaped GEMM on the gfx950 matrix cores: C = ep(to16(beta * A @ B)).
//
// One kernel serves every weight kind the reference multiplies on its dense
// f16/bf16 MOPA path:
//   - Q4 (matmul_q4 / matmul_q4_bf16 for m > 8): replaces run_q4_panels +
//     unpack_q4_f16 (csrc/gemm_f16f16_q4.h:57-118) and the bf16 twin
//     (csrc/gemm_b16b16_q4.h:32);
//   - Q2 / Q1 (matmul_q2_mopa / matmul_q1_mopa): replaces unpack_q{1,2}_f16 +
//     lowbit_panels (csrc/gemm_f16f16_lowbit.h:27-194);
//   - dense Packed<f16> / Packed<bf16> (Gemm::new(&a, &packed, m)...run()):
//     replaces run_packed (csrc/gemm_half.h:1054).
// Weight tiles are dequantized straight into LDS as f16/bf16 (each weight
// rounded once, exactly as the reference's dequant: q4/mod.rs:193-224,
// lowbit/matmul.rs:178-197), then multiplied with v_mfma_f32_16x16x32_{f16,bf16}
// accumulating in f32 -- the portable path's accumulator type
// (src/reference.rs:349-387). The store rounds beta*acc to 16 bits and runs the
// op-graph on that value (src/exec/macros.rs:188-206).
//
// Tiling: 128x128 output tile per 256-thread workgroup (2x2 waves of 64x64),
// K steps of 64 depths, LDS double-buffered so the next tile's global loads
// and dequant overlap the current tile's MFMAs.
#include "kernels.h"

namespace smg {

namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // halfs per LDS row (pad against bank conflicts)
constexpr int TILE_HALFS = 128 * LDS_STRIDE;

struct GemmArgs {
    const uint16_t *lhs;
    uint16_t *dst;
    const uint8_t *codes;
    const uint16_t *sc;
    const uint16_t *mn;
    const uint16_t *dense;
    long lhs_rs, lhs_cs, dst_rs, dst_cs;
    uint32_t m, n, k, n_pad, nchunks, k_pad;
    uint32_t block_shift;
    uint32_t codebook;
    float beta;
    uint32_t lhs_bytes;  // byte footprint of A (the buffer resource's range)
    uint32_t vec_a;      // A rows 16-byte aligned, unit column stride, k % 8 == 0
};

template <bool BF16>
__device__ __forceinline__ float4_t mfma(const uint4 &a, const uint4 &b, float4_t c) {
    if (!BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
    } else {
        typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
}

// ---- B-tile staging: global -> registers (issued early) -> LDS (dequant) ----
//
// Each thread owns one "unit" of the 128-column x 64-depth B tile; the unit's
// shape depends on the weight kind:
//   Q4:    column t%128, 32 depths (one 16-byte chunk), chunk t/128 of the step
//   Q2:    column t%128, 32 depths (8 bytes: half a chunk)
//   Q1:    column t%128, 32 depths (4 bytes: a quarter chunk)
//   dense: column t/2, 32 depths (64 bytes)
struct BRegs {
    uint4 raw[4];
    uint16_t s, mn;
};

template <int WK>
__device__ __forceinline__ void b_load(const GemmArgs &g, uint32_t col0, uint32_t k0, BRegs &r) {
    const int t = threadIdx.x;
    if (WK == W_F16 || WK == W_BF16) {
        const uint32_t col = col0 + t / 2;
        const uint32_t d = k0 + (t % 2) * 32;
        const uint4 *p = (const uint4 *)(g.dense + (size_t)col * g.k_pad + d);
#pragma unroll
        for (int q = 0; q < 4; q++) r.raw[q] = p[q];
        return;
    }
    const uint32_t col = col0 + t % 128;
    const uint32_t d = k0 + (t / 128) * 32;  // first depth of the unit
    constexpr uint32_t CH = WK == W_Q4 ? Q4_CHUNK : WK == W_Q2 ? Q2_GROUP : Q1_GROUP;
    // Branch-free: a chunk past K loads the last chunk (a valid address) and
    // its scale is forced to 0, so its weights are +-0. (Low-bit groups cover
    // K in multiples of 256 depths, so only Q4 ever has a dead chunk.)
    const uint32_t kc = d / CH;
    const bool live = kc < g.nchunks;
    const uint32_t kcc = live ? kc : g.nchunks - 1;
    const uint32_t dc = kcc * CH + d % CH;
    r.raw[0] = make_uint4(0, 0, 0, 0);
    if (WK == W_Q4) {
        r.raw[0] = *(const uint4 *)(g.codes + ((size_t)kcc * g.n_pad + col) * 16);
    } else {
        // quarters g and g+1 of the unit's slab: two dwords 16 bytes apart
        const uint8_t *p = g.codes + lb_dword_offset<WK == W_Q2 ? 2 : 1>(dc, col, g.n_pad);
        r.raw[0].x = *(const uint32_t *)p;
        r.raw[0].y = *(const uint32_t *)(p + 16);
    }
    r.s = 0;
    r.mn = 0;
    if (g.block_shift >= 5) {
        const uint32_t kb = dc >> g.block_shift;
        const uint16_t s = g.sc[(size_t)kb * g.n_pad + col];
        r.s = live ? s : (uint16_t)0;
        if (WK == W_Q4 && g.mn) {
            const uint16_t mv = g.mn[(size_t)kb * g.n_pad + col];
            r.mn = live ? mv : (uint16_t)0;
        }
    }
}

// Write one unit into the LDS B tile (column-major: B_lds[col][depth]).
template <int WK, bool BF16, bool AFFINE>
__device__ __forceinline__ void b_store(const GemmArgs &g, uint32_t col0, uint32_t k0,
                                        const BRegs &r, uint16_t *blds) {
    const int t = threadIdx.x;
    if (WK == W_F16 || WK == W_BF16) {
        uint16_t *dstp = blds + (t / 2) * LDS_STRIDE + (t % 2) * 32;
#pragma unroll
        for (int q = 0; q < 4; q++) *(uint4 *)(dstp + q * 8) = r.raw[q];
        return;
    }
    const int cl = t % 128;
    const int dl = (t / 128) * 32;
    const uint32_t col = col0 + cl;
    const uint32_t d0 = k0 + dl;
    uint16_t *dstp = blds + cl * LDS_STRIDE + dl;
    uint32_t out[16];
    if (WK == W_Q4) {
        const uint32_t words[4] = {r.raw[0].x, r.raw[0].y, r.raw[0].z, r.raw[0].w};
        const bool fast = !BF16 && !AFFINE && g.block_shift >= 5;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t q = words[w];  // stored nibbles are code + 8
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t u = (q >> (4 * e)) & 0x000F000Fu;
                if (fast) {
                    half2_t h = __builtin_bit_cast(half2_t, u | 0x64006400u);
                    const half2_t magic = {(_Float16)1032.0f, (_Float16)1032.0f};
                    _Float16 s = __builtin_bit_cast(_Float16, r.s);
                    half2_t s2 = {s, s};
                    out[w * 4 + e] = __builtin_bit_cast(uint32_t, (h - magic) * s2);
                } else {
                    const int c0 = (int)(u & 0xF) - 8, c1 = (int)(u >> 16) - 8;
                    const uint32_t dp = d0 + w * 8 + 2 * e;
                    uint16_t s0 = r.s, s1 = r.s, m0 = r.mn, m1 = r.mn;
                    if (g.block_shift < 5) {
                        const uint32_t b0 = dp >> g.block_shift, b1 = (dp + 1) >> g.block_shift;
                        s0 = g.sc[(size_t)b0 * g.n_pad + col];
                        s1 = g.sc[(size_t)b1 * g.n_pad + col];
                        if (AFFINE) {
                            m0 = g.mn[(size_t)b0 * g.n_pad + col];
                            m1 = g.mn[(size_t)b1 * g.n_pad + col];
                        }
                    }
                    uint16_t w0, w1;
                    if (!AFFINE) {
                        w0 = from_f32<BF16>(f16_to_f32(s0) * (float)c0);
                        w1 = from_f32<BF16>(f16_to_f32(s1) * (float)c1);
                    } else {
                        const double v0 = (double)f16_to_f32(s0) * (double)c0 + (double)f16_to_f32(m0);
                        const double v1 = (double)f16_to_f32(s1) * (double)c1 + (double)f16_to_f32(m1);
                        w0 = BF16 ? f32_to_bf16((float)v0) : f64_to_f16(v0);
                        w1 = BF16 ? f32_to_bf16((float)v1) : f64_to_f16(v1);
                    }
                    out[w * 4 + e] = (uint32_t)w0 | ((uint32_t)w1 << 16);
                }
            }
        }
    } else if (WK == W_Q2) {
        // f16(scale * codebook[code]): the product is exact in f32 (matmul.rs:185-187)
        const uint32_t words[2] = {r.raw[0].x, r.raw[0].y};
#pragma unroll
        for (int w = 0; w < 2; w++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t sel = (words[w] >> (2 * i)) & 0x03030303u;
                const uint32_t vals = __builtin_amdgcn_perm(g.codebook, g.codebook, sel);
                uint16_t h[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const uint32_t dp = d0 + w * 16 + 4 * i + b;
                    const uint16_t sb = g.block_shift >= 5
                                            ? r.s
                                            : g.sc[(size_t)(dp >> g.block_shift) * g.n_pad + col];
                    const float v = (float)(int8_t)(vals >> (8 * b));
                    h[b] = f32_to_f16(f16_to_f32(sb) * v);
                }
                out[w * 8 + 2 * i] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
                out[w * 8 + 2 * i + 1] = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            }
        }
    } else {
        // Q1: +scale for a set bit, -scale otherwise (exact). Each dword holds
        // two slabs; this unit's slab is bit-half hs.
        const uint32_t words[2] = {r.raw[0].x, r.raw[0].y};
        const uint32_t hs = ((d0 % Q1_GROUP) / LB_SLAB) % 2;
#pragma unroll
        for (int w = 0; w < 2; w++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t bits = (words[w] >> (4 * hs + i)) & 0x01010101u;
                uint16_t h[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const uint32_t dp = d0 + w * 16 + 4 * i + b;
                    const uint16_t sb = g.block_shift >= 5
                                            ? r.s
                                            : g.sc[(size_t)(dp >> g.block_shift) * g.n_pad + col];
                    const uint32_t bit = (bits >> (8 * b)) & 1u;
                    h[b] = bit ? sb : (uint16_t)(sb ^ 0x8000u);
                }
                out[w * 8 + 2 * i] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
                out[w * 8 + 2 * i + 1] = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            }
        }
    }
    // Q1/Q2 depth order inside out[]: depth 4i+b sits at half-word 4i+b, i.e.
    // natural order. Q4: depth 8w+2e+h at half-word 8w+2e+h, also natural.
#pragma unroll
    for (int q = 0; q < 4; q++)
        *(uint4 *)(dstp + q * 8) = make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
}

// ---- A-tile staging: 128 rows x 64 depths; thread t: row t/2, 32 depths ----
__device__ __forceinline__ void a_load(const GemmArgs &g, uint32_t row0, uint32_t k0,
                                       uint4 (&ra)[4]) {
    // buffer loads: out-of-range offsets read zero, no branches
    const int t = threadIdx.x;
    const uint32_t row = row0 + t / 2;
    const uint32_t d = k0 + (t % 2) * 32;
    const rsrc_t rs = make_rsrc(g.lhs, g.lhs_bytes);
    if (g.vec_a) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            ra[q] = bload16(rs, (row < g.m && d + 8 * q < g.k)
                                    ? (uint32_t)(row * g.lhs_rs + d + 8 * q) * 2u
                                    : OOB);
        return;
    }
    uint16_t e[32];
#pragma unroll
    for (int q = 0; q < 32; q++)
        e[q] = bload2(rs, (row < g.m && d + q < g.k)
                              ? (uint32_t)(row * g.lhs_rs + (d + q) * g.lhs_cs) * 2u
                              : OOB);
#pragma unroll
    for (int q = 0; q < 4; q++)
        ra[q] = make_uint4(e[8 * q] | ((uint32_t)e[8 * q + 1] << 16),
                           e[8 * q + 2] | ((uint32_t)e[8 * q + 3] << 16),
                           e[8 * q + 4] | ((uint32_t)e[8 * q + 5] << 16),
                           e[8 * q + 6] | ((uint32_t)e[8 * q + 7] << 16));
}

__device__ __forceinline__ void a_store(const uint4 (&ra)[4], uint16_t *alds) {
    const int t = threadIdx.x;
    uint16_t *dstp = alds + (t / 2) * LDS_STRIDE + (t % 2) * 32;
#pragma unroll
    for (int q = 0; q < 4; q++) *(uint4 *)(dstp + q * 8) = ra[q];
}

template <int WK, bool BF16, bool AFFINE>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs g, EpArgs ep) {
    extern __shared__ __align__(16) uint16_t lds[];
    // stage s: A at lds + 2*s*TILE, B at lds + (2*s+1)*TILE

    // column-tile-major grid order: consecutive workgroups share a weight tile
    const uint32_t mtiles = (g.m + BM - 1) / BM;
    const uint32_t tile = blockIdx.x;
    const uint32_t tm = tile % mtiles, tn = tile / mtiles;
    const uint32_t row0 = tm * BM, col0 = tn * BN;

    const int t = threadIdx.x;
    const int lane = t % 64, wave = t / 64;
    const int wm = wave / 2, wn = wave % 2;
    const int lr = lane % 16, lk = (lane / 16) * 8;

    float4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jt = 0; jt < 4; jt++) acc[i][jt] = (float4_t){0.f, 0.f, 0.f, 0.f};

    const uint32_t ksteps = (g.k + BK - 1) / BK;
    uint4 ra[4];
    BRegs rb;
    a_load(g, row0, 0, ra);
    b_load<WK>(g, col0, 0, rb);
    a_store(ra, lds);
    b_store<WK, BF16, AFFINE>(g, col0, 0, rb, lds + TILE_HALFS);
    __syncthreads();

    for (uint32_t ks = 0; ks < ksteps; ks++) {
        const int cur = ks & 1;
        const bool more = ks + 1 < ksteps;
        if (more) {
            a_load(g, row0, (ks + 1) * BK, ra);
            b_load<WK>(g, col0, (ks + 1) * BK, rb);
        }
        const uint16_t *Al = lds + 2 * cur * TILE_HALFS;
        const uint16_t *Bl = Al + TILE_HALFS;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            uint4 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = *(const uint4 *)(Al + (wm * 64 + i * 16 + lr) * LDS_STRIDE + kk + lk);
#pragma unroll
            for (int jt = 0; jt < 4; jt++)
                bf[jt] = *(const uint4 *)(Bl + (wn * 64 + jt * 16 + lr) * LDS_STRIDE + kk + lk);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jt = 0; jt < 4; jt++) acc[i][jt] = mfma<BF16>(af[i], bf[jt], acc[i][jt]);
        }
        if (more) {
            uint16_t *An = lds + 2 * (cur ^ 1) * TILE_HALFS;
            a_store(ra, An);
            b_store<WK, BF16, AFFINE>(g, col0, (ks + 1) * BK, rb, An + TILE_HALFS);
        }
        __syncthreads();
    }

    // store: lane holds D[4*(lane/16)+v][lane%16] of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jt = 0; jt < 4; jt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const uint32_t row = row0 + wm * 64 + i * 16 + (lane / 16) * 4 + v;
                const uint32_t col = col0 + wn * 64 + jt * 16 + lr;
                if (row < g.m && col < g.n) {
                    const float x = 0.0f + g.beta * acc[i][jt][v];
                    g.dst[(size_t)row * g.dst_rs + (size_t)col * g.dst_cs] =
                        finish<BF16>(ep, x, row, col, g.n);
                }
            }
}

template <int WK, bool BF16, bool AFFINE>
hipError_t launch_t(const GemmArgs &g, const EpArgs &ep, hipStream_t s) {
    const size_t lds = 4 * TILE_HALFS * 2;
    static bool attr_set = false;  // benign race: every setter writes the same value
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)gemm_kernel<WK, BF16, AFFINE>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t tiles = ((g.m + BM - 1) / BM) * ((g.n + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_kernel<WK, BF16, AFFINE>), dim3(tiles), dim3(256), lds, s, g, ep);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                       const uint16_t *lhs, long lhs_cs, long lhs_rs, float beta,
                       const EpArgs &ep, bool bf16, hipStream_t s) {
    GemmArgs g = {};
    g.lhs = lhs;
    g.dst = dst;
    g.codes = w.codes;
    g.sc = w.scales;
    g.mn = w.mins;
    g.dense = w.dense;
    g.lhs_rs = lhs_rs;
    g.lhs_cs = lhs_cs;
    g.dst_rs = dst_rs;
    g.dst_cs = dst_cs;
    g.m = (uint32_t)m;
    g.n = (uint32_t)w.n;
    g.k = (uint32_t)w.k;
    g.n_pad = (uint32_t)w.n_pad;
    g.nchunks = (uint32_t)w.nchunks;
    g.k_pad = (uint32_t)w.k_pad;
    g.block_shift = w.block ? (uint32_t)__builtin_ctzll(w.block) : 0;
    g.codebook = w.codebook;
    g.beta = beta;
    const size_t fp = (m && w.k) ? ((m - 1) * (size_t)lhs_rs + (w.k - 1) * (size_t)lhs_cs + 1) * 2 : 0;
    if (fp >= ((size_t)1 << 31)) return hipErrorInvalidValue;  // one buffer resource spans < 2 GiB
    g.lhs_bytes = (uint32_t)fp;
    g.vec_a = (lhs_cs == 1 && lhs_rs % 8 == 0 && w.k % 8 == 0 &&
               ((uintptr_t)lhs & 15) == 0) ? 1u : 0u;
    const bool affine = w.mins != nullptr;
    switch (w.kind) {
    case W_Q4:
        if (bf16) return affine ? launch_t<W_Q4, true, true>(g, ep, s) : launch_t<W_Q4, true, false>(g, ep, s);
        return affine ? launch_t<W_Q4, false, true>(g, ep, s) : launch_t<W_Q4, false, false>(g, ep, s);
    case W_Q2: return launch_t<W_Q2, false, false>(g, ep, s);
    case W_Q1: return launch_t<W_Q1, false, false>(g, ep, s);
    case W_F16: return launch_t<W_F16, false, false>(g, ep, s);
    case W_BF16: return launch_t<W_BF16, true, false>(g, ep, s);
    default: return hipErrorInvalidValue;
    }
}

// Eager dequant of Q4 weights to the dense layout ([n_pad][k_pad], column's K
// contiguous), one thread per (column, 32-depth chunk).
namespace {
template <bool BF16, bool AFFINE>
__global__ void q4_dequant_kernel(WDev w, uint16_t *dense) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t kcs = w.k_pad / 32;
    if (idx >= w.n_pad * kcs) return;
    const size_t col = idx / kcs, kc = idx % kcs;
    uint16_t *out = dense + col * w.k_pad + kc * 32;
    if (col >= w.n || kc >= w.nchunks) {
        for (int q = 0; q < 32; q++) out[q] = 0;
        return;
    }
    const uint4 raw = *(const uint4 *)(w.codes + (kc * w.n_pad + col) * 16);
    const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
    const uint32_t shift = (uint32_t)__builtin_ctzll(w.block);
    for (int wd = 0; wd < 4; wd++) {
        const uint32_t q = words[wd];  // stored nibbles are code + 8
        for (int e = 0; e < 4; e++) {
            const uint32_t u = (q >> (4 * e)) & 0x000F000Fu;
            const int cs[2] = {(int)(u & 0xF) - 8, (int)(u >> 16) - 8};
            for (int h = 0; h < 2; h++) {
                const size_t d = kc * 32 + wd * 8 + 2 * e + h;
                uint16_t v = 0;
                if (d < w.k) {
                    const size_t kb = d >> shift;
                    const float s = f16_to_f32(w.scales[kb * w.n_pad + col]);
                    if (!AFFINE) {
                        v = from_f32<BF16>(s * (float)cs[h]);
                    } else {
                        const double x = (double)s * (double)cs[h] +
                                         (double)f16_to_f32(w.mins[kb * w.n_pad + col]);
                        v = BF16 ? f32_to_bf16((float)x) : f64_to_f16(x);
                    }
                }
                out[wd * 8 + 2 * e + h] = v;
            }
        }
    }
}
}  // namespace

hipError_t launch_q4_dequant_dense(const WDev &q4, uint16_t *dense, bool to_bf16, hipStream_t s) {
    WDev w = q4;
    const size_t total = w.n_pad * (w.k_pad / 32);
    const dim3 grid((unsigned)((total + 255) / 256));
    const bool affine = w.mins != nullptr;
    if (to_bf16) {
        if (affine) hipLaunchKernelGGL((q4_dequant_kernel<true, true>), grid, dim3(256), 0, s, w, dense);
        else hipLaunchKernelGGL((q4_dequant_kernel<true, false>), grid, dim3(256), 0, s, w, dense);
    } else {
        if (affine) hipLaunchKernelGGL((q4_dequant_kernel<false, true>), grid, dim3(256), 0, s, w, dense);
        else hipLaunchKernelGGL((q4_dequant_kernel<false, false>), grid, dim3(256), 0, s, w, dense);
    }
    return hipGetLastError();
}

}  // namespace smg
