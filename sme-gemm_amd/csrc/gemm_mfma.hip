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
// Tiling: BM x 128 output tile (BM = 256 with 8 waves, or 128 with 4 waves),
// every wave a 64 x 64 sub-tile, K in steps of 64 depths. Two register stages
// and two LDS buffers: the global loads for step k+2 are issued while step k
// multiplies, and step k+1 is dequantized into the other LDS buffer at the end
// of step k, so each load has two steps of MFMA work to arrive behind. With
// BM = 256 every Q4 weight is dequantized once per 256 output rows.
#include <algorithm>

#include "kernels.h"
#include "tile_store.cuh"

namespace smg {

namespace {

constexpr int BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK;  // halfs per LDS row: 8 chunks of 16 bytes, swizzled

// 16-byte chunk c of LDS row r lives at chunk c ^ (r & 7) of that row, so the
// rows a fragment read or a tile store touches together hit different banks.
__device__ __forceinline__ int swz(int row, int chunk) { return row * LDS_STRIDE + ((chunk ^ (row & 7)) << 3); }

struct GemmArgs {
    const uint16_t *lhs;
    uint16_t *dst;
    const uint8_t *codes;
    const uint16_t *sc;
    const uint16_t *mn;
    const uint16_t *dense;
    long lhs_rs, lhs_cs, dst_rs, dst_cs;
    uint32_t m, n, k, n_pad, nchunks, k_pad;
    uint32_t sc_rows;  // rows of the scale (and min) grids
    uint32_t block_shift;
    uint32_t codebook;
    float beta;
    float alpha;         // read_dst: C = alpha * C + beta * A@B
    uint32_t read_dst;
    uint32_t lhs_bytes;  // byte footprint of A (the buffer resource's range)
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

// ---- B tile: global -> registers (early) -> LDS (dequantized) ----------------
// Thread t owns column t % 128 and UD consecutive depths (t / 128) * UD of the
// 128-column x 64-depth tile; UD = 64 * 128 / threads (32 or 16).
template <int UD>
struct BRegs {
    // dense: UD halfs; Q4 uses dwords 0..UD/8-1, low-bit dwords 0..UD/16-1.
    // A vector type (not an array) so the register stages never go to scratch.
    uint32_t __attribute__((ext_vector_type(UD / 2))) v;
    uint16_t s, mn;
    uint32_t dc;  // first depth actually loaded (clamped into the weights)
    bool live;    // false for a unit past K: its weights are forced to 0
};

template <int WK, int UD>
__device__ __forceinline__ void b_load(const GemmArgs &g, uint32_t col0, uint32_t k0, BRegs<UD> &r) {
    const int t = threadIdx.x;
    const uint32_t col = col0 + t % 128;
    const uint32_t d = k0 + (t / 128) * UD;  // first depth of the unit
    if constexpr (WK == W_F16 || WK == W_BF16) {
        r.live = d < g.k_pad;
        const uint4 *p = (const uint4 *)(g.dense + (size_t)col * g.k_pad + (r.live ? d : g.k_pad - UD));
#pragma unroll
        for (int q = 0; q < UD / 8; q++) {
            const uint4 x = p[q];
            r.v[4 * q] = x.x;
            r.v[4 * q + 1] = x.y;
            r.v[4 * q + 2] = x.z;
            r.v[4 * q + 3] = x.w;
        }
        return;
    }
    constexpr uint32_t CH = WK == W_Q4 ? Q4_CHUNK : WK == W_Q2 ? Q2_GROUP : Q1_GROUP;
    // Branch-free: a unit past K (a padding chunk, or a step issued past the
    // last one) loads from the last chunk (a valid address) and its scale is
    // forced to 0 in b_store, so its weights are +-0.
    const uint32_t kc = d / CH;
    const bool live = kc < g.nchunks;
    const uint32_t kcc = live ? kc : g.nchunks - 1;
    const uint32_t dc = kcc * CH + d % CH;
    if constexpr (WK == W_Q4) {
        const uint8_t *p = g.codes + cell_index(kcc, col, g.nchunks, g.n_pad) * 16 + ((d % 32) / 8) * 4;
        if constexpr (UD == 32) {
            const uint4 x = *(const uint4 *)p;
            r.v[0] = x.x;
            r.v[1] = x.y;
            r.v[2] = x.z;
            r.v[3] = x.w;
        } else {
            const uint2 x = *(const uint2 *)p;
            r.v[0] = x.x;
            r.v[1] = x.y;
        }
    } else {
        // quarter(s) of the unit's slab: dwords 16 bytes apart
        const uint8_t *p = g.codes + lb_dword_offset<WK == W_Q2 ? 2 : 1>(dc, col, g.nchunks, g.n_pad);
        r.v[0] = *(const uint32_t *)p;
        if constexpr (UD == 32) r.v[1] = *(const uint32_t *)(p + 16);
    }
    // Scale (and min) loads are unconditional so no wait is forced here: the
    // values are only consumed (and masked by `live`) in b_store. When the
    // block is shorter than the unit, b_store reads per-depth scales instead.
    const size_t si = cell_index(dc >> g.block_shift, col, g.sc_rows, g.n_pad);
    r.s = g.sc[si];
    if constexpr (WK == W_Q4) r.mn = (g.mn ? g.mn : g.sc)[si];
    r.live = live;
    r.dc = dc;
}

// PD: blocks shorter than a thread's UD depths, so scales vary per depth
// (a separate instantiation keeps that rare path out of the common kernel).
template <int WK, bool BF16, bool AFFINE, int UD, bool PD>
__device__ __forceinline__ void b_store(const GemmArgs &g, uint32_t col0, const BRegs<UD> &r, uint16_t *blds) {
    const int t = threadIdx.x;
    const int cl = t % 128;
    const int dl = (t / 128) * UD;
    if constexpr (WK == W_F16 || WK == W_BF16) {
#pragma unroll
        for (int q = 0; q < UD / 8; q++)
            *(uint4 *)(blds + swz(cl, dl / 8 + q)) =
                r.live ? make_uint4(r.v[4 * q], r.v[4 * q + 1], r.v[4 * q + 2], r.v[4 * q + 3])
                       : make_uint4(0, 0, 0, 0);
        return;
    }
    const uint32_t col = col0 + cl;
    const uint32_t d0 = r.dc;  // per-depth scales are read at clamped depths
    constexpr bool per_depth = PD;  // scale per depth
    const uint16_t us = r.live ? r.s : (uint16_t)0;
    const uint16_t um = r.live ? r.mn : (uint16_t)0;
    uint32_t out[UD / 2];
    if constexpr (WK == W_Q4) {
        const uint32_t words[4] = {r.v[0], r.v[1], r.v[2], r.v[3]};
        const bool fast = !BF16 && !AFFINE && !per_depth;
        const uint32_t mag_lo = 0x64006400u, mag_hi = 0x54005400u;
#pragma unroll
        for (int w = 0; w < UD / 8; w++) {
            const uint32_t q = words[w];  // stored nibbles are code + 8
            if (fast) {
                // bfi puts the nibble under an f16 exponent; subtracting the
                // bias leaves the exact code; one multiply rounds scale*code
                const _Float16 s = __builtin_bit_cast(_Float16, us);
                const half2_t s2 = {s, s};
                const half2_t off_lo = {(_Float16)1032.0f, (_Float16)1032.0f};
                const half2_t off_hi = {(_Float16)72.0f, (_Float16)72.0f};
                const uint32_t q8 = q >> 8;
                out[w * 4 + 0] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, bfi(0x000F000Fu, q, mag_lo)) - off_lo) * s2);
                out[w * 4 + 1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, bfi(0x00F000F0u, q, mag_hi)) - off_hi) * s2);
                out[w * 4 + 2] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, bfi(0x000F000Fu, q8, mag_lo)) - off_lo) * s2);
                out[w * 4 + 3] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, bfi(0x00F000F0u, q8, mag_hi)) - off_hi) * s2);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t u = (q >> (4 * e)) & 0x000F000Fu;
                    const int c0 = (int)(u & 0xF) - 8, c1 = (int)(u >> 16) - 8;
                    const uint32_t dp = d0 + w * 8 + 2 * e;
                    uint16_t s0 = us, s1 = us, m0 = um, m1 = um;
                    if (per_depth) {
                        const uint32_t b0 = dp >> g.block_shift, b1 = (dp + 1) >> g.block_shift;
                        s0 = r.live ? g.sc[cell_index(b0, col, g.sc_rows, g.n_pad)] : (uint16_t)0;
                        s1 = r.live ? g.sc[cell_index(b1, col, g.sc_rows, g.n_pad)] : (uint16_t)0;
                        if (AFFINE) {
                            m0 = r.live ? g.mn[cell_index(b0, col, g.sc_rows, g.n_pad)] : (uint16_t)0;
                            m1 = r.live ? g.mn[cell_index(b1, col, g.sc_rows, g.n_pad)] : (uint16_t)0;
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
    } else if constexpr (WK == W_Q2) {
        // f16(scale * codebook[code]): the product is exact in f32 (matmul.rs:185-187)
        const uint32_t words[2] = {r.v[0], r.v[1]};
#pragma unroll
        for (int w = 0; w < UD / 16; w++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t sel = (words[w] >> (2 * i)) & 0x03030303u;
                const uint32_t vals = __builtin_amdgcn_perm(g.codebook, g.codebook, sel);
                uint16_t h[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const uint32_t dp = d0 + w * 16 + 4 * i + b;
                    const uint16_t sb = per_depth ? (r.live ? g.sc[cell_index(dp >> g.block_shift, col, g.sc_rows, g.n_pad)] : (uint16_t)0) : us;
                    h[b] = f32_to_f16(f16_to_f32(sb) * (float)(int8_t)(vals >> (8 * b)));
                }
                out[w * 8 + 2 * i] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
                out[w * 8 + 2 * i + 1] = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            }
        }
    } else {
        // Q1: +scale for a set bit, -scale otherwise (exact). Each dword holds
        // two slabs; this unit's slab is bit-half hs.
        const uint32_t words[2] = {r.v[0], r.v[1]};
        const uint32_t hs = ((d0 % Q1_GROUP) / LB_SLAB) % 2;
#pragma unroll
        for (int w = 0; w < UD / 16; w++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t bits = (words[w] >> (4 * hs + i)) & 0x01010101u;
                uint16_t h[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const uint32_t dp = d0 + w * 16 + 4 * i + b;
                    const uint16_t sb = per_depth ? (r.live ? g.sc[cell_index(dp >> g.block_shift, col, g.sc_rows, g.n_pad)] : (uint16_t)0) : us;
                    h[b] = ((bits >> (8 * b)) & 1u) ? sb : (uint16_t)(sb ^ 0x8000u);
                }
                out[w * 8 + 2 * i] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
                out[w * 8 + 2 * i + 1] = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            }
        }
    }
    // depth order inside out[]: natural (depth x at half-word x)
#pragma unroll
    for (int q = 0; q < UD / 8; q++)
        *(uint4 *)(blds + swz(cl, dl / 8 + q)) = make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
}

// ---- A tile: BM rows x 64 depths; thread t: row t/2, 32 depths --------------
template <bool VECA>
__device__ __forceinline__ void a_load(const GemmArgs &g, uint32_t row0, uint32_t k0, uint4 (&ra)[4]) {
    // buffer loads: out-of-range offsets read zero, no branches
    const int t = threadIdx.x;
    const uint32_t row = row0 + t / 2;
    const uint32_t d = k0 + (t % 2) * 32;
    const rsrc_t rs = make_rsrc(g.lhs, g.lhs_bytes);
    if constexpr (VECA) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            ra[q] = bload16(rs, (row < g.m && d + 8 * q < g.k)
                                    ? (uint32_t)(row * g.lhs_rs + d + 8 * q) * 2u : OOB);
        return;
    }
    uint16_t e[32];
#pragma unroll
    for (int q = 0; q < 32; q++)
        e[q] = bload2(rs, (row < g.m && d + q < g.k)
                              ? (uint32_t)(row * g.lhs_rs + (d + q) * g.lhs_cs) * 2u : OOB);
#pragma unroll
    for (int q = 0; q < 4; q++)
        ra[q] = make_uint4(e[8 * q] | ((uint32_t)e[8 * q + 1] << 16),
                           e[8 * q + 2] | ((uint32_t)e[8 * q + 3] << 16),
                           e[8 * q + 4] | ((uint32_t)e[8 * q + 5] << 16),
                           e[8 * q + 6] | ((uint32_t)e[8 * q + 7] << 16));
}

__device__ __forceinline__ void a_store(const uint4 (&ra)[4], uint16_t *alds) {
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; q++) *(uint4 *)(alds + swz(t / 2, (t % 2) * 4 + q)) = ra[q];
}

// One 32-depth half of a step's fragments (A: 4 row blocks, B: 4 column
// blocks of the wave's 64 x 64 sub-tile), and its 16 products.
template <int BM>
__device__ __forceinline__ void read_half(const uint16_t *stage, int kk, int wm, int wn, int lane,
                                          uint4 (&fa)[4], uint4 (&fb)[4]) {
    const uint16_t *Bl = stage + BM * LDS_STRIDE;
    const int lr = lane % 16, ch = kk / 8 + lane / 16;
#pragma unroll
    for (int i = 0; i < 4; i++) fa[i] = *(const uint4 *)(stage + swz(wm * 64 + i * 16 + lr, ch));
#pragma unroll
    for (int jt = 0; jt < 4; jt++) fb[jt] = *(const uint4 *)(Bl + swz(wn * 64 + jt * 16 + lr, ch));
}

template <bool BF16>
__device__ __forceinline__ void mma_half(const uint4 (&fa)[4], const uint4 (&fb)[4], float4_t (&acc)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jt = 0; jt < 4; jt++) acc[i][jt] = mfma<BF16>(fa[i], fb[jt], acc[i][jt]);
}

// The tile store shared by the GEMM kernels. acc holds the wave's 64 x 64
// sub-tile (wave (wm, wn) of the BM x 128 tile); the loop's last barrier has
// freed the LDS.
template <bool BF16, int BM>
__device__ __forceinline__ void store_tile(const GemmArgs &g, const EpArgs &ep, const float4_t (&acc)[4][4],
                                           uint16_t *lds, uint32_t row0, uint32_t col0, int wm, int wn,
                                           int lane) {
    const int t = threadIdx.x, lr = lane % 16;
    // Round beta*acc to 16 bits into LDS (the loop's last barrier freed it); a
    // lane holds D[4*(lane/16)+v][lane%16] of each 16x16 MFMA tile. The LDS
    // holds BM * CS halfs of tile plus the operand vectors (EPI_LDS_HALFS).
    // With read_dst and no op-graph the old C joins before the one rounding,
    // alpha * C + beta * acc in f32 (src/reference.rs:349-387); with a graph
    // it is added after the graph (ep_store8).
    constexpr int CS = BN + 8;  // halfs per staged row
    const bool rd_here = g.read_dst && ep.n_nodes == 0;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jt = 0; jt < 4; jt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int rl = wm * 64 + i * 16 + (lane / 16) * 4 + v, cl = wn * 64 + jt * 16 + lr;
                float prev = 0.0f;
                if (rd_here && row0 + rl < g.m && col0 + cl < g.n)
                    prev = g.alpha * to_f32<BF16>(g.dst[(size_t)(row0 + rl) * g.dst_rs + (size_t)(col0 + cl) * g.dst_cs]);
                lds[rl * CS + cl] = from_f32<BF16>(prev + g.beta * acc[i][jt][v]);
            }
    __syncthreads();
    const StoreArgs sa = {g.dst, g.dst_rs, g.dst_cs, g.m, g.n, g.alpha, g.read_dst && ep.n_nodes != 0};
    float *colv = (float *)(lds + BM * CS);      // [node][BN]
    float *rowv = colv + EP_FUSED * BN;  // [node][BM]
    ep_load_vectors<BF16, BM, BN, BM * 2>(sa, ep, colv, rowv, row0, col0);
    __syncthreads();
    for (int u = t; u < BM * (BN / 8); u += BM * 2) {
        const int rl = u / (BN / 8), cl = (u % (BN / 8)) * 8;
        ep_store8<BF16, BM, BN>(sa, ep, colv, rowv, *(const uint4 *)(lds + rl * CS + cl), rl, cl, row0, col0);
    }
}

constexpr int EPI_LDS_HALFS(int bm) { return bm * (BN + 8) + EP_FUSED * (BN + bm) * 2; }

template <int BM>
struct Tile {
    static constexpr int THREADS = BM * 2;          // BM/64 x 2 waves
    static constexpr int UD = 64 * 128 / THREADS;   // B depths per thread
    static constexpr int STAGE = (BM + BN) * LDS_STRIDE;  // halfs per LDS stage
    static constexpr int NSTAGE = 3;                // LDS ring
    static_assert(EPI_LDS_HALFS(BM) <= NSTAGE * STAGE, "the tile store exceeds the LDS ring");
};

template <int WK, bool BF16, bool AFFINE, int BM, bool VECA, bool PD>
__global__ void __launch_bounds__(BM * 2) gemm_kernel(GemmArgs g, EpArgs ep) {
    constexpr int UD = Tile<BM>::UD;
    constexpr int STAGE = Tile<BM>::STAGE;
    extern __shared__ __align__(16) uint16_t lds[];  // [3][A: BM rows | B: 128 rows] x 64, swizzled

    // column-tile-major order: consecutive workgroups share a weight tile
    const uint32_t mtiles = (g.m + BM - 1) / BM;
    const uint32_t tile = xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t tm = tile % mtiles, tn = tile / mtiles;
    const uint32_t row0 = tm * BM, col0 = tn * BN;

    const int t = threadIdx.x;
    const int lane = t % 64, wave = t / 64;
    const int wm = wave / 2, wn = wave % 2;

    float4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jt = 0; jt < 4; jt++) acc[i][jt] = (float4_t){0.f, 0.f, 0.f, 0.f};

    uint4 ra0[4], ra1[4];
    BRegs<UD> rb0, rb1;

    // Pipeline, per 64-depth step k: the global loads of step k+3 are issued,
    // step k+2 is dequantized into LDS stage (k+2)%3, and the fragments of
    // step k+1 are read from stage (k+1)%3 -- published by the barrier that
    // ended step k-1 -- while step k multiplies. Every load is unconditional
    // (steps past K read zeros, see b_load and a_load), so the compiler counts
    // outstanding loads exactly. The step count is rounded up to even (two
    // register stages); an odd count multiplies one zero step.
    const uint32_t ksteps = (g.k + 2 * BK - 1) / (2 * BK) * 2;  // >= 2
    a_load<VECA>(g, row0, 0, ra0);
    b_load<WK, UD>(g, col0, 0, rb0);
    a_load<VECA>(g, row0, BK, ra1);
    b_load<WK, UD>(g, col0, BK, rb1);
    a_store(ra0, lds);
    b_store<WK, BF16, AFFINE, UD, PD>(g, col0, rb0, lds + BM * LDS_STRIDE);
    a_load<VECA>(g, row0, 2 * BK, ra0);
    b_load<WK, UD>(g, col0, 2 * BK, rb0);
    a_store(ra1, lds + STAGE);
    b_store<WK, BF16, AFFINE, UD, PD>(g, col0, rb1, lds + STAGE + BM * LDS_STRIDE);
    __syncthreads();

    uint4 fa0[4], fb0[4], fa1[4], fb1[4];  // kk = 0 / kk = 32 halves
    read_half<BM>(lds, 0, wm, wn, lane, fa0, fb0);
    uint32_t s_cur = 0;  // stage of step ks
    for (uint32_t ks = 0; ks < ksteps; ks += 2) {
        // even step ks: its second half, the next step's first half, step
        // ks+3's loads into register stage 1, step ks+2 (stage 0) into LDS
        {
            const uint32_t s1 = s_cur == 2 ? 0 : s_cur + 1, s2 = s1 == 2 ? 0 : s1 + 1;
            read_half<BM>(lds + s_cur * STAGE, 32, wm, wn, lane, fa1, fb1);
            mma_half<BF16>(fa0, fb0, acc);
            read_half<BM>(lds + s1 * STAGE, 0, wm, wn, lane, fa0, fb0);
            a_load<VECA>(g, row0, (ks + 3) * BK, ra1);
            b_load<WK, UD>(g, col0, (ks + 3) * BK, rb1);
            a_store(ra0, lds + s2 * STAGE);
            b_store<WK, BF16, AFFINE, UD, PD>(g, col0, rb0, lds + s2 * STAGE + BM * LDS_STRIDE);
            mma_half<BF16>(fa1, fb1, acc);
            __syncthreads();
            s_cur = s1;
        }
        // odd step ks+1: the same with the register stages swapped
        {
            const uint32_t s1 = s_cur == 2 ? 0 : s_cur + 1, s2 = s1 == 2 ? 0 : s1 + 1;
            read_half<BM>(lds + s_cur * STAGE, 32, wm, wn, lane, fa1, fb1);
            mma_half<BF16>(fa0, fb0, acc);
            read_half<BM>(lds + s1 * STAGE, 0, wm, wn, lane, fa0, fb0);
            a_load<VECA>(g, row0, (ks + 4) * BK, ra0);
            b_load<WK, UD>(g, col0, (ks + 4) * BK, rb0);
            a_store(ra1, lds + s2 * STAGE);
            b_store<WK, BF16, AFFINE, UD, PD>(g, col0, rb1, lds + s2 * STAGE + BM * LDS_STRIDE);
            mma_half<BF16>(fa1, fb1, acc);
            __syncthreads();
            s_cur = s1;
        }
    }

    store_tile<BF16, BM>(g, ep, acc, lds, row0, col0, wm, wn, lane);
}

template <int WK, bool BF16, bool AFFINE, int BM, bool VECA, bool PD>
hipError_t launch_t(const GemmArgs &g, const EpArgs &ep, hipStream_t s) {
    const size_t lds = (size_t)Tile<BM>::NSTAGE * Tile<BM>::STAGE * 2;
    static bool attr_set = false;  // benign race: every setter writes the same value
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute((const void *)gemm_kernel<WK, BF16, AFFINE, BM, VECA, PD>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t tiles = ((g.m + BM - 1) / BM) * ((g.n + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_kernel<WK, BF16, AFFINE, BM, VECA, PD>), dim3(tiles), dim3(BM * 2), lds, s,
                       g, ep);
    return hipGetLastError();
}

template <int WK, bool BF16, bool AFFINE>
hipError_t launch_shape(const GemmArgs &g, const EpArgs &ep, bool vec_a, hipStream_t s) {
    const uint32_t block = 1u << g.block_shift;
    if constexpr (WK == W_Q4 || WK == W_Q2 || WK == W_Q1) {
        if (!vec_a)
            return block < 32 ? launch_t<WK, BF16, AFFINE, 128, false, true>(g, ep, s)
                              : launch_t<WK, BF16, AFFINE, 128, false, false>(g, ep, s);
        if (g.m > 128)
            return block < 16 ? launch_t<WK, BF16, AFFINE, 256, true, true>(g, ep, s)
                              : launch_t<WK, BF16, AFFINE, 256, true, false>(g, ep, s);
        return block < 32 ? launch_t<WK, BF16, AFFINE, 128, true, true>(g, ep, s)
                          : launch_t<WK, BF16, AFFINE, 128, true, false>(g, ep, s);
    } else {
        (void)block;
        if (!vec_a) return launch_t<WK, BF16, AFFINE, 128, false, false>(g, ep, s);
        if (g.m > 128) return launch_t<WK, BF16, AFFINE, 256, true, false>(g, ep, s);
        return launch_t<WK, BF16, AFFINE, 128, true, false>(g, ep, s);
    }
}

// An op-graph longer than a store's EP_FUSED nodes, as a pass over C: cell
// (i, j) of src is the product rounded to T, stored without a graph, and
// dst[i, j] = to16(graph(f32(src[i, j]))) in the node order of ep_cell (a
// trailing activation rounded once) -- with add_dst, to16(f32(that) + alpha *
// f32(old dst[i, j])), the store's add_dst step. src is dst unless add_dst.
template <bool BF16>
__global__ void __launch_bounds__(256) ep_tail(const uint16_t *src, long src_rs, long src_cs, uint16_t *dst,
                                               long dst_rs, long dst_cs, uint32_t m, uint32_t n, float alpha,
                                               uint32_t add_dst, EpLong ep) {
    const size_t total = (size_t)m * n;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
        const uint32_t i = (uint32_t)(idx / n), j = (uint32_t)(idx % n);
        const uint16_t c = src[(size_t)i * src_rs + (size_t)j * src_cs];
        uint16_t out = ep_cell<BF16>(ep, to_f32<BF16>(c), i, j, n);
        uint16_t *dp = dst + (size_t)i * dst_rs + (size_t)j * dst_cs;
        if (add_dst) out = from_f32<BF16>(to_f32<BF16>(out) + alpha * to_f32<BF16>(*dp));
        *dp = out;
    }
}

}  // namespace

hipError_t launch_ep_tail(const uint16_t *src, long src_rs, long src_cs, uint16_t *dst, long dst_rs, long dst_cs,
                          size_t m, size_t n, float alpha, bool add_dst, const EpLong &ep, bool bf16, hipStream_t s) {
    if (m == 0 || n == 0 || ep.n_nodes == 0) return hipSuccess;
    if (m > 0xFFFFFFFFu || n > 0xFFFFFFFFu) return hipErrorInvalidValue;
    const size_t blocks = std::min<size_t>(((size_t)m * n + 255) / 256, (size_t)1 << 20);
    if (bf16)
        hipLaunchKernelGGL(ep_tail<true>, dim3((uint32_t)blocks), dim3(256), 0, s, src, src_rs, src_cs, dst, dst_rs,
                           dst_cs, (uint32_t)m, (uint32_t)n, alpha, add_dst ? 1u : 0u, ep);
    else
        hipLaunchKernelGGL(ep_tail<false>, dim3((uint32_t)blocks), dim3(256), 0, s, src, src_rs, src_cs, dst, dst_rs,
                           dst_cs, (uint32_t)m, (uint32_t)n, alpha, add_dst ? 1u : 0u, ep);
    return hipGetLastError();
}

hipError_t launch_gemm(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                       const uint16_t *lhs, long lhs_cs, long lhs_rs, float beta,
                       const EpArgs &ep, bool bf16, hipStream_t s, bool read_dst, float alpha) {
    if (read_dst && w.kind != W_F16 && w.kind != W_BF16) return hipErrorInvalidValue;
    if (!read_dst && q4r_supported(w, m, lhs_cs, lhs_rs, lhs, bf16))
        return launch_q4r(w, m, dst, dst_cs, dst_rs, lhs, lhs_rs, beta, ep, nullptr, 0, bf16, s);
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
    g.sc_rows = (uint32_t)w.sc_rows;
    g.k_pad = (uint32_t)w.k_pad;
    g.block_shift = w.block ? (uint32_t)__builtin_ctzll(w.block) : 0;
    g.codebook = w.codebook;
    g.beta = beta;
    g.alpha = alpha;
    g.read_dst = read_dst ? 1u : 0u;
    const size_t fp = (m && w.k) ? ((m - 1) * (size_t)lhs_rs + (w.k - 1) * (size_t)lhs_cs + 1) * 2 : 0;
    if (fp >= ((size_t)1 << 31)) return hipErrorInvalidValue;  // one buffer resource spans < 2 GiB
    g.lhs_bytes = (uint32_t)fp;
    const bool vec_a = lhs_cs == 1 && lhs_rs % 8 == 0 && w.k % 8 == 0 && ((uintptr_t)lhs & 15) == 0;
    const bool affine = w.mins != nullptr;
    switch (w.kind) {
    case W_Q4:
        if (bf16) return affine ? launch_shape<W_Q4, true, true>(g, ep, vec_a, s) : launch_shape<W_Q4, true, false>(g, ep, vec_a, s);
        return affine ? launch_shape<W_Q4, false, true>(g, ep, vec_a, s) : launch_shape<W_Q4, false, false>(g, ep, vec_a, s);
    case W_Q2: return launch_shape<W_Q2, false, false>(g, ep, vec_a, s);
    case W_Q1: return launch_shape<W_Q1, false, false>(g, ep, vec_a, s);
    case W_F16: return launch_shape<W_F16, false, false>(g, ep, vec_a, s);
    case W_BF16: return launch_shape<W_BF16, true, false>(g, ep, vec_a, s);
    default: return hipErrorInvalidValue;
    }
}

// A strided k x n B into the dense layout, 32 x 32 blocks through LDS: the
// reads run along whichever of B's two strides is 1 when the block's threads
// walk j (a row-major B) and the writes along the dense column's K.
namespace {
__global__ void __launch_bounds__(256) pack_dense_strided(const uint16_t *rhs, long rhs_rs, long rhs_cs,
                                                          uint32_t n, uint32_t k, uint32_t k_pad,
                                                          uint16_t *dense) {
    __shared__ uint16_t tile[32][33];
    const uint32_t l0 = blockIdx.x * 32, j0 = blockIdx.y * 32;
    const uint32_t tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 32 x 8
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t l = l0 + ty + 8 * r, j = j0 + tx;
        tile[ty + 8 * r][tx] = (l < k && j < n) ? rhs[(long)l * rhs_rs + (long)j * rhs_cs] : (uint16_t)0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t j = j0 + ty + 8 * r, l = l0 + tx;
        if (l < k_pad) dense[(size_t)j * k_pad + l] = tile[tx][ty + 8 * r];
    }
}
}  // namespace

hipError_t launch_pack_dense_strided(const uint16_t *rhs, long rhs_rs, long rhs_cs, size_t n, size_t k,
                                     size_t n_pad, size_t k_pad, uint16_t *dense, hipStream_t s) {
    if (n_pad % 32 || k_pad % 32 || n > n_pad || k > k_pad) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(k_pad / 32), (unsigned)(n_pad / 32));
    hipLaunchKernelGGL(pack_dense_strided, grid, dim3(256), 0, s, rhs, rhs_rs, rhs_cs, (uint32_t)n, (uint32_t)k,
                       (uint32_t)k_pad, dense);
    return hipGetLastError();
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
    const uint4 raw = *(const uint4 *)(w.codes + cell_index(kc, col, w.nchunks, w.n_pad) * 16);
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
                    const float s = f16_to_f32(w.scales[cell_index(kb, col, w.sc_rows, w.n_pad)]);
                    if (!AFFINE) {
                        v = from_f32<BF16>(s * (float)cs[h]);
                    } else {
                        const double x = (double)s * (double)cs[h] +
                                         (double)f16_to_f32(w.mins[cell_index(kb, col, w.sc_rows, w.n_pad)]);
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
