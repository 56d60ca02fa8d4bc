// 2-bit / 1-bit int8 GEMV: matmul_q2 / matmul_q1 (+ _ep).
//
// Replaces csrc/gemm_q2.cc:48-429 (q2_quant, run_q2_gemv, Q2_FOLD) and gives
// the reference's portable result bit for bit (src/kernels/lowbit/matmul.rs:354-398):
//   1. each row of A is quantized per K-block: amax = max|a| (NaN if any a is),
//      inv = amax > 0 ? 127/amax : 0, s = amax/127 (IEEE divides),
//      q = round_ties_even(a*inv) saturated to int8 (NaN -> 0);
//   2. exact i32 block sums sum_d q_d * value(d, j), value = codebook[code]
//      (Q2) or +-1 (Q1);
//   3. per output, in block order: total = fmaf(f32(sum), f32(scale)*s, total)
//      with the product scale*s rounded on its own;
//   4. f16 RNE, then the op-graph.
//
// Two kernels per call:
// lowbit_quant: one workgroup per (row, block): q (int8), s and sum(q) into a
//   small device buffer (the activations are read once, not once per column
//   tile).
// lowbit_gemv: a workgroup of 8 waves owns 16 output columns; the K-blocks of a
//   segment are split into 8 contiguous ranges, one per wave. A wave computes
//   each of its blocks' sums on v_mfma_i32_16x16x64_i8 (exact i32): A operand =
//   16 columns x 64 depths of weights expanded to int8 (Q2: one v_perm_b32 per
//   4 depths with the codebook bytes as the table; Q1: sign bits to 0/1 bytes,
//   using sum(q*(2b-1)) = 2*sum(q*b) - sum(q)), B operand = 64 depths x up to 16
//   rows of q. Sums go to LDS; then one lane per output folds them in block
//   order -- the only sequential step, and it is one fma per block.
#include <algorithm>
#include <type_traits>

#include "kernels.h"

namespace smg {

namespace {

constexpr int WV = 8;          // waves per workgroup
constexpr int T = WV * 64;
constexpr int MAXS = 8;        // 64-depth slabs per wave per segment (weight registers)
constexpr int S_BUDGET = 65536;  // LDS bytes of block sums per segment

struct LbArgs {
    const uint8_t *codes;
    const uint16_t *sc;
    uint16_t *dst;
    const int8_t *q;      // [m][kq] quantized activations
    const float *s;       // [m][nbq] activation block scales
    const int32_t *asum;  // [m][nbq] block sums of q
    uint32_t n, k, n_pad, m;
    uint32_t block_shift;
    uint32_t codebook;
    uint32_t kq, nbq;     // row strides of q and of s / asum
    uint32_t sc_rows;
    uint32_t ngroups;     // 16-byte code groups per column (rows of the code grid)
    uint32_t seg_depths;  // depths per segment (a multiple of max(block, 64))
};

template <int KIND, int MR>
__global__ void __launch_bounds__(T) lowbit_gemv(LbArgs g, EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t block = 1u << g.block_shift;
    // block slots per segment (1 when blocks are longer than a segment)
    const uint32_t nbs = g.seg_depths >= block ? g.seg_depths >> g.block_shift : 1;
    int32_t *S = (int32_t *)smem;                        // [nbs][16][MR]
    uint16_t *scl = (uint16_t *)(smem + (size_t)nbs * 16 * MR * 4);  // [nbs][16]
    float *sa = (float *)(scl + nbs * 16);               // [MR][nbs]
    int32_t *as = (int32_t *)(sa + MR * nbs);            // [MR][nbs]

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int gq4 = lane >> 4, c = lane & 15;   // quarter; column (A) / row (B)
    const uint32_t col0 = xcd_tile(blockIdx.x, gridDim.x) * 16;
    const uint32_t col = col0 + c;               // < n_pad
    const uint32_t row0 = blockIdx.y * MR;
    const uint32_t mr = min((uint32_t)MR, g.m - row0);

    const rsrc_t qr = make_rsrc(g.q, g.m * g.kq);
    const rsrc_t sr = make_rsrc(g.sc, (uint32_t)cell_grid_rows(g.sc_rows) * g.n_pad * 2u);
    const rsrc_t fr = make_rsrc(g.s, g.m * g.nbq * 4u);
    const rsrc_t ur = make_rsrc(g.asum, g.m * g.nbq * 4u);

    // fold lanes: (column fc, row frow)
    const int fc = t & 15, frow = t >> 4;
    const bool folder = frow < MR && (uint32_t)frow < mr;
    float total = 0.0f;

    const uint32_t nseg = (g.k + g.seg_depths - 1) / g.seg_depths;
    for (uint32_t seg = 0; seg < nseg; seg++) {
        const uint32_t d0 = seg * g.seg_depths;
        const uint32_t dl = min(g.seg_depths, g.k - d0);
        // blocks overlapping the segment; a block longer than a segment keeps
        // its slot-0 partial sum from the segment before
        const uint32_t b0 = d0 >> g.block_shift;
        const uint32_t nb = ((d0 + dl - 1) >> g.block_shift) - b0 + 1;
        const bool carry = (d0 & (block - 1)) != 0;
        const bool block_done = ((d0 + dl) & (block - 1)) == 0 || d0 + dl == g.k;
        // this wave's contiguous slab range
        const uint32_t nslab = (dl + LB_SLAB - 1) / LB_SLAB;
        const uint32_t sa0 = d0 / LB_SLAB + (nslab * wave) / WV;
        const uint32_t ns = (nslab * (wave + 1)) / WV - (nslab * wave) / WV;  // <= MAXS
        // -- 1. loads: activations (B operand), weights (A operand), then the
        //       fold's scales; all in flight before anything waits
        uint4 qreg[MAXS];
        uint32_t wreg[MAXS];
#pragma unroll
        for (int i = 0; i < MAXS; i++) {
            const uint32_t slab = sa0 + i;
            const bool live = (uint32_t)i < ns;
            qreg[i] = bload16(qr, (live && (uint32_t)c < mr)
                                      ? (row0 + c) * g.kq + slab * LB_SLAB + 16 * gq4 : OOB);
            const uint32_t sl = live ? slab : sa0;  // dead slots reload a valid dword
            wreg[i] = *(const uint32_t *)(g.codes +
                                          lb_dword_offset<KIND>((size_t)sl * LB_SLAB + 16 * gq4, col, g.ngroups, g.n_pad));
        }
        // scales of the 16 columns (32 bytes a block), activation scales, sums
        constexpr int RS = 4;  // up to 4 x 512 x 16 B = 32 KB of scale rows
        uint4 sreg[RS];
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const uint32_t i = t + T * r, bb = i / 2, half = i % 2;
            sreg[r] = bload16(sr, bb < nb ? (uint32_t)cell_index(b0 + bb, col0, g.sc_rows, g.n_pad) * 2u + half * 16u : OOB);
        }
        float fsa[2];
        int32_t fas[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint32_t i = t + T * r, rr = i / nbs, bb = i % nbs;
            const bool ok = rr < mr && bb < nb && i < MR * nbs;
            fsa[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                fr, ok ? ((row0 + rr) * g.nbq + b0 + bb) * 4u : OOB, 0, 0));
            fas[r] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(
                ur, ok ? ((row0 + rr) * g.nbq + b0 + bb) * 4u : OOB, 0, 0);
        }
        // zero the block sums (not a carried slot)
        for (uint32_t i = t; i < nbs * 16 * MR; i += T)
            if (!(carry && i < 16 * MR)) S[i] = 0;
        __syncthreads();
        // -- 2. block sums on the matrix cores; partial sums of a block split
        //       between waves meet in LDS through integer atomics (exact)
        const uint32_t parts = block < (uint32_t)LB_SLAB ? LB_SLAB / block : 1;
        const uint32_t spb = block > (uint32_t)LB_SLAB ? block / LB_SLAB : 1;  // slabs per block
        int4_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < MAXS; i++) {
            if ((uint32_t)i < ns) {  // uniform
                const uint32_t slab = sa0 + i;
                int4_t wa;
                if (KIND == 2) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        wa[j] = (int)__builtin_amdgcn_perm(g.codebook, g.codebook,
                                                           (wreg[i] >> (2 * j)) & 0x03030303u);
                } else {
                    const uint32_t hs = 4 * (((slab * LB_SLAB) % Q1_GROUP) / LB_SLAB % 2);
#pragma unroll
                    for (int j = 0; j < 4; j++) wa[j] = (int)((wreg[i] >> (hs + j)) & 0x01010101u);
                }
                const int4_t ab = __builtin_bit_cast(int4_t, qreg[i]);
                for (uint32_t p = 0; p < parts; p++) {
                    int4_t abp = ab;
                    if (parts > 1 && (uint32_t)(16 * gq4) / block != p) abp = (int4_t){0, 0, 0, 0};
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, abp, acc, 0, 0, 0);
                    // flush at a block's end or at the end of this wave's range
                    const bool flush = parts > 1 || ((slab + 1) % spb) == 0 || (uint32_t)i + 1 == ns;
                    if (flush) {  // uniform
                        const uint32_t bl =
                            ((slab * LB_SLAB + p * (parts > 1 ? block : 0)) >> g.block_shift) - b0;
                        if ((uint32_t)c < mr) {
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                atomicAdd(&S[(bl * 16 + 4 * gq4 + v) * MR + c], acc[v]);
                        }
                        acc = (int4_t){0, 0, 0, 0};
                    }
                }
            }
        }
        // -- 3. stage the fold's operands, then fold the finished blocks in order
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const uint32_t i = t + T * r, bb = i / 2, half = i % 2;
            if (bb < nb) *(uint4 *)(scl + bb * 16 + half * 8) = sreg[r];
        }
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint32_t i = t + T * r;
            if (i < MR * nbs) {
                sa[i] = fsa[r];
                as[i] = fas[r];
            }
        }
        __syncthreads();
        if (folder) {
            // the last block waits for its remaining depths when it continues
            const uint32_t nfold = block_done ? nb : nb - 1;
            for (uint32_t bb = 0; bb < nfold; bb++) {
                int32_t sum = S[(bb * 16 + fc) * MR + frow];
                if (KIND == 1) sum = 2 * sum - as[frow * nbs + bb];
                const float scv = f16_to_f32(scl[bb * 16 + fc]) * sa[frow * nbs + bb];
                total = fmaf((float)sum, scv, total);
            }
        }
        __syncthreads();
    }
    if (folder) {
        const uint32_t row = row0 + frow, j = col0 + fc;
        if (j < g.n) g.dst[(size_t)row * g.n + j] = finish<false>(ep, total, row, j, g.n);
    }
}

// ---------------------------------------------------------------------------
// Single-launch path (m <= 8, block <= 4096, K <= 8192, m*K <= 32 K): one
// workgroup of 8 waves per 16*CG-column tile, a straight-line program kept
// short (each workgroup runs it once, so its instruction fetch is part of the
// latency). With one row, each workgroup quantizes A itself -- 8 KB read from
// L2 -- so a call is one launch; with more rows that work would repeat in every
// workgroup, so lowbit_prequant quantizes them once before the launch and the
// workgroups load the result:
//   1. loads: A (or its quantized rows), then the scale rows, the epilogue
//      operands and the tile's code groups (a wave covers a contiguous K range
//      in whole 16-byte groups: Q2 4 slabs, Q1 8);
//   2. quantize (quant_pass): thread t takes depths 8t..8t+7 (per 4096-depth
//      pass) of every row; a block's amax and sum(q) are reduced over the
//      block's lanes by shuffles, and through LDS over waves for blocks longer
//      than 512;
//   3. exact block sums on v_mfma_i32_16x16x64_i8, accumulated over a block's
//      slabs inside one wave (a wave's K range holds whole blocks; shorter
//      blocks take one masked product each), written to LDS per (row, column)
//      with blocks contiguous;
//   4. every thread turns a few (row, column, block) sums into the fold's two
//      factors, f32(sum) and f32(scale)*s, so that
//   5. one lane per output folds its blocks in order with fmaf -- four LDS
//      loads and 16 fmas per 16 blocks, the one sequential step, after the
//      bytes have arrived -- then the op-graph and the f16 store.
// LDS rows are padded so these accesses do not collide on banks.
// ---------------------------------------------------------------------------
constexpr uint32_t QPASS = T * 8;  // depths quantized per pass (8 per thread)

struct LtArgs {
    const uint8_t *codes;
    const uint16_t *sc;
    const uint16_t *lhs;
    uint16_t *dst;
    uint32_t n, k, n_pad, m;
    uint32_t block_shift;
    uint32_t codebook;
    uint32_t sc_rows;
    uint32_t ngroups;      // 16-byte code groups per column
    uint32_t kq;           // depths the waves cover (8 waves x NG groups)
    uint32_t nbq;          // blocks in kq (a multiple of 4)
    uint32_t codes_bytes;  // extent of the code array (buffer resource)
    uint32_t cg_shift;     // log2 of the 16-column groups per workgroup (CG)
    // rows quantized beforehand by lowbit_prequant (multi-row calls):
    const int8_t *q;       // [m][kq]
    const float *qs;       // [m][nbq] activation block scales
    const int32_t *qsum;   // [m][nbq] negated block sums of q
};

__device__ __forceinline__ float nanmax(float a, float b) {
    return (a != a) ? a : ((b != b) ? b : fmaxf(a, b));
}
// Reductions over aligned groups of gl lanes (gl a power of two <= 64): DPP
// within 16-lane rows (quad swaps, then the half-row and row mirrors pair
// each lane with one from the other half), cross-lane shuffles beyond.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
// (The DPP moves zero their out-of-row lanes, bound_ctrl, which these row
// permutations never read: the compiler then folds each move into the max or
// add that consumes it.)
template <int CTRL>
__device__ __forceinline__ uint32_t dppz(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t group_max_u32(uint32_t a, uint32_t gl) {
    if (gl > 1) a = max(a, dppz<0xB1>(a));   // quad_perm [1,0,3,2]
    if (gl > 2) a = max(a, dppz<0x4E>(a));   // quad_perm [2,3,0,1]
    if (gl > 4) a = max(a, dppz<0x141>(a));  // row_half_mirror
    if (gl > 8) a = max(a, dppz<0x140>(a));  // row_mirror
    if (gl > 16) a = max(a, (uint32_t)__shfl_xor((int)a, 16));
    if (gl > 32) a = max(a, (uint32_t)__shfl_xor((int)a, 32));
    return a;
}
__device__ __forceinline__ int32_t group_sum_i32(int32_t a, uint32_t gl) {
    if (gl > 1) a += (int32_t)dppz<0xB1>((uint32_t)a);
    if (gl > 2) a += (int32_t)dppz<0x4E>((uint32_t)a);
    if (gl > 4) a += (int32_t)dppz<0x141>((uint32_t)a);
    if (gl > 8) a += (int32_t)dppz<0x140>((uint32_t)a);
    if (gl > 16) a += __shfl_xor(a, 16);
    if (gl > 32) a += __shfl_xor(a, 32);
    return a;
}

// Four f16 activations (two dwords) quantized with the block's inv and packed
// into four int8 bytes: f32(a) * inv with one rounding (v_fma_mix_f32: the f16
// operand widened exactly, a -0 addend leaves the product as it is), ties to
// even (v_rndne_f32), then v_cvt_i32_f32, whose NaN gives 0 as the reference's
// quantize_row does. No clamp is needed: |a| <= amax, inv <= 127/amax * (1 +
// 2^-24), so |a * inv| rounds to at most 127 (and inv = 0 when amax is 0, inf
// or NaN, leaving 0 or NaN).
__device__ __forceinline__ uint32_t quant4(uint32_t w0, uint32_t w1, float inv) {
    float f[4];
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(f[0]) : "v"(w0), "v"(inv), "v"(-0.0f));
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(f[1]) : "v"(w0), "v"(inv), "v"(-0.0f));
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(f[2]) : "v"(w1), "v"(inv), "v"(-0.0f));
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(f[3]) : "v"(w1), "v"(inv), "v"(-0.0f));
    uint32_t q[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float r = __builtin_rintf(f[e]);
        asm("v_cvt_i32_f32 %0, %1" : "=v"(q[e]) : "v"(r));
    }
    const uint32_t lo = __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u);  // {q0, q1, 0, 0} (low bytes)
    const uint32_t hi = __builtin_amdgcn_perm(q[3], q[2], 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// LDS: q [MR][kq + 16] i8, for one row later the fold's y and x, each [16
//      CG][nbq + 4] f32 (the products have read q by then) | s [MR][nbq] f32 |
//      -sum(q) [MR][nbq] i32 | block sums [MR][16 CG][nbq + 4] i32 (one row:
//      [nbq][16 CG], a lane's four columns in one 16-byte store) | scales [16
//      CG][nbq + 4] f16 | wave partials
__host__ __device__ inline uint32_t tile_q_region(uint32_t kq, uint32_t nbq, uint32_t mr, uint32_t cg) {
    const uint32_t q = mr * (kq + 16), xy = mr == 1 ? 2 * 16 * cg * (nbq + 4) * 4 : 0;
    return q > xy ? q : xy;
}
// The one-row layout for blocks of 128 (fast, the usual decode call): q [kq
// + 16] i8 | 64 zero bytes | s [nbq] f32 | -sum(q) [nbq] i32 | the fold's (x,
// y) pairs [16 CG][nbq + 2] | wave partials.
size_t tile_lds_bytes(uint32_t kq, uint32_t nbq, int mr, uint32_t cg, bool fast) {
    if (fast) return (size_t)kq + 16 + 64 + (size_t)nbq * 8 + (size_t)16 * cg * (nbq + 2) * 8 + (size_t)WV * 8;
    return (size_t)tile_q_region(kq, nbq, (uint32_t)mr, cg) + (size_t)mr * nbq * 8 +
           (size_t)mr * 16 * cg * (nbq + 4) * 4 + (size_t)16 * cg * (nbq + 4) * 2 + (size_t)mr * WV * 8;
}

// One 4096-depth pass of quantize_row (src/kernels/lowbit/matmul.rs:354-371)
// over MR rows: thread t holds depths p*4096 + 8t .. +7 of each row in ar[r];
// q goes to q + r*qstride + depth, the block's s and -sum(q) to
// s[r*nbq + block], sum[r*nbq + block] (-sum(q) only for Q1, whose fold adds
// it to 2*sum(q*b)).
// A block's amax and sum(q) reduce over its lanes by DPP / shuffles, and
// through the LDS words wmax / wsum ([MR][WV]) for blocks longer than 512.
// BSH: the block's log2 when fixed at compile time (7: blocks of 128, the
// usual decode format), 0 for the runtime block_shift.
template <int KIND, int MR, int BSH = 0>
__device__ __forceinline__ void quant_pass(const uint4 (&ar)[MR], uint32_t p, int8_t *q, uint32_t qstride,
                                           float *s, int32_t *sum_out, uint32_t nbq, uint32_t kq,
                                           uint32_t block_shift, float *wmax, int32_t *wsum) {
    typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if constexpr (BSH > 0) block_shift = BSH;
    const uint32_t block = 1u << block_shift;
    const uint32_t gl = block / 8 < 64u ? block / 8 : 64u;  // lanes of a block in a wave
    const uint32_t wpb = block > 512u ? block / 512u : 1u;   // waves of a block
    const uint32_t d0 = p * QPASS + 8 * t;
    // |a| as f16 magnitude bits: their unsigned order is the numeric order,
    // and every NaN pattern sorts above infinity, so an integer max is the
    // reference's NaN-propagating amax
    float am[MR];
#pragma unroll
    for (int r = 0; r < MR; r++) {
        const u16x2_t w0 = __builtin_bit_cast(u16x2_t, ar[r].x & 0x7FFF7FFFu);
        const u16x2_t w1 = __builtin_bit_cast(u16x2_t, ar[r].y & 0x7FFF7FFFu);
        const u16x2_t w2 = __builtin_bit_cast(u16x2_t, ar[r].z & 0x7FFF7FFFu);
        const u16x2_t w3 = __builtin_bit_cast(u16x2_t, ar[r].w & 0x7FFF7FFFu);
        const u16x2_t mx = __builtin_elementwise_max(__builtin_elementwise_max(w0, w1),
                                                     __builtin_elementwise_max(w2, w3));
        am[r] = f16_to_f32((uint16_t)group_max_u32(max((uint32_t)mx.x, (uint32_t)mx.y), gl));
    }
    if (wpb > 1) {  // blocks longer than a wave: combine the waves' maxima
        if (p > 0) __syncthreads();
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < MR; r++) wmax[r * WV + wave] = am[r];
        __syncthreads();
        const uint32_t w0 = (wave / wpb) * wpb;
#pragma unroll
        for (int r = 0; r < MR; r++) {
            float a = 0.0f;
            for (uint32_t w = 0; w < wpb; w++) a = nanmax(a, wmax[r * WV + w0 + w]);
            am[r] = a;
        }
    }
    int32_t qs[MR];
#pragma unroll
    for (int r = 0; r < MR; r++) {
        const float inv = am[r] > 0.0f ? __fdiv_rn(127.0f, am[r]) : 0.0f;
        const uint32_t qw0 = quant4(ar[r].x, ar[r].y, inv), qw1 = quant4(ar[r].z, ar[r].w, inv);
        if (d0 < kq) *(uint2 *)(q + r * qstride + d0) = make_uint2(qw0, qw1);
        if constexpr (KIND == 1) {
            const int32_t sum = __builtin_amdgcn_sdot4((int)qw1, 0x01010101, __builtin_amdgcn_sdot4((int)qw0, 0x01010101, 0, false), false);
            qs[r] = group_sum_i32(sum, gl);
        } else {
            qs[r] = 0;
        }
    }
    if (KIND == 1 && wpb > 1) {
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < MR; r++) wsum[r * WV + wave] = qs[r];
        __syncthreads();
        const uint32_t w0 = (wave / wpb) * wpb;
#pragma unroll
        for (int r = 0; r < MR; r++) {
            int32_t sum = 0;
            for (uint32_t w = 0; w < wpb; w++) sum += wsum[r * WV + w0 + w];
            qs[r] = sum;
        }
    }
    if ((uint32_t)lane % gl == 0 && (uint32_t)wave % wpb == 0 && d0 < kq) {
        const uint32_t bb = d0 >> block_shift;
#pragma unroll
        for (int r = 0; r < MR; r++) {
            s[r * nbq + bb] = __fdiv_rn(am[r], 127.0f);
            sum_out[r * nbq + bb] = -qs[r];
        }
    }
}

// The multi-row single-launch path quantizes A once per call, here, instead of
// once per workgroup: one workgroup per (4096-depth pass, row) writes q
// [m][kq] (zero past k) and the blocks' s and -sum(q) [m][nbq].
template <int KIND>
__global__ void __launch_bounds__(T) lowbit_prequant(const uint16_t *lhs, uint32_t m, uint32_t k,
                                                     uint32_t kq, uint32_t nbq, uint32_t block_shift,
                                                     int8_t *q, float *s, int32_t *sum) {
    __shared__ float wmax[WV];
    __shared__ int32_t wsum[WV];
    const uint32_t p = blockIdx.x, r = blockIdx.y;
    const rsrc_t ar = make_rsrc(lhs, m * k * 2u);
    const uint4 a[1] = {load_row8(ar, r, m, k, p * QPASS + 8 * threadIdx.x, (k & 7) == 0)};
    quant_pass<KIND, 1>(a, p, q + (size_t)r * kq, 0, s + (size_t)r * nbq, sum + (size_t)r * nbq, nbq, kq,
                        block_shift, wmax, wsum);
}

// SPB: slabs per block when fixed at compile time (2 = blocks of 128, the
// usual decode format), 0 for any block (runtime block structure).
// EPV: the store's op-graph, compiled for the common shapes (the host picks
// it from the graph): 0 any graph (ep), 1 none, 2 add_col(col_b) then a
// trailing activation act (0: none, alpha its scalar), 3 mul_col(col_a),
// add_col(col_b), then act. Each runs the graph's f32 steps in its order on
// the f16-rounded sum, as the generic store does.
// The first 14 argument dwords arrive in SGPRs with the wave (this file is
// compiled with kernarg preloading): everything but col_a, alpha and the
// interpreted graph, so no scalar load of an argument sits on the kernel's
// path. The rest derive from them: misc = m | block_shift << 8 | cg_shift <<
// 16 | act << 24; n_pad = n rounded up to 128 (every weight handle's grid);
// the code groups per column, ceil(k / group depths); src is A (f16 [m][k],
// one row) or its pre-quantized rows (int8 [m][kq], several), followed by
// their block scales and negated sums (lowbit_prequant's layout).
template <int KIND, int MR, int NG, int SPB, int EPV>
__global__ void __launch_bounds__(T)
    lowbit_tile(const uint8_t *codes, const uint16_t *sc, const void *src, uint16_t *dst, const uint16_t *col_b,
                uint32_t k, uint32_t misc, uint32_t n, uint32_t codebook, const uint16_t *col_a, float alpha,
                EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr uint32_t SPG = KIND == 2 ? 4 : 8;  // slabs per code group
    constexpr int NSW = NG * (int)SPG;            // slabs per wave
    constexpr int QP = 2;                         // A passes held in registers (K <= 8192)
    constexpr int PQ = 4;                         // pre-quantized block entries per thread
    // SPB 2: blocks of 128 (the host launches SPB 2 only for them)
    const uint32_t m = misc & 0xFF, block_shift = SPB == 2 ? 7u : (misc >> 8) & 0xFF;
    const uint32_t cg_shift = (misc >> 16) & 0xFF, act = misc >> 24;
    const uint32_t n_pad = ((n ? n : 1u) + 127u) & ~127u;
    const uint32_t tiles = n_pad >> (4 + cg_shift);
    const uint32_t block = 1u << block_shift;
    // the host's geometry (tile_geometry_cg): 8 / CG waves along K cover kq
    const uint32_t kq = (8u >> cg_shift) * NSW * LB_SLAB;
    const uint32_t nbq = ((kq >> block_shift) + 3) & ~3u;
    const uint32_t grp_depths = KIND == 2 ? Q2_GROUP : Q1_GROUP;
    const uint32_t ngroups = (k + grp_depths - 1) / grp_depths;
    const uint32_t sc_rows = (ngroups * grp_depths + block - 1) >> block_shift;
    const uint32_t cg = 1u << cg_shift;           // 16-column groups in this workgroup
    const uint32_t ncol = 16 * cg;
    const uint32_t qs_ = kq + 16;   // q row stride (bytes)
    const uint32_t bs = nbq + 4;    // block-sum / scale row stride (elements)
    // FAST: one row, blocks of 128 (tile_lds_bytes' fast layout). Each wave's
    // products put block b of its range in row b of the MFMA output (the B
    // operand's column b holds q on that block's slabs, zeros elsewhere), so
    // the lanes that hold a block's sums form the fold's factors right after
    // the products, with the scales they loaded themselves.
    constexpr bool FAST = MR == 1 && SPB == 2;
    constexpr int NBW = SPB > 0 ? NSW / SPB : 1;  // blocks per wave (SPB > 0)
    static_assert(!FAST || NBW <= 16, "a wave's blocks are rows of one product tile");
    const uint32_t bs2 = nbq + 2;   // (x, y) pair row stride (FAST)
    int8_t *ql = (int8_t *)smem;                        // [MR][qs_]
    const int8_t *zq = ql + qs_;                        // 64 zero bytes (FAST)
    float *yl = (float *)smem;                          // [ncol][bs] (one row), after the products
    float *xl = yl + ncol * bs;                         // [ncol][bs] (one row), after the products
    float *sa = (float *)(smem + (FAST ? qs_ + 64 : tile_q_region(kq, nbq, MR, cg)));  // [MR][nbq]
    int32_t *as = (int32_t *)(sa + MR * nbq);           // [MR][nbq]
    float2 *xy = (float2 *)(as + MR * nbq);             // [ncol][bs2] (FAST)
    int32_t *sb = as + MR * nbq;                        // [MR][ncol][bs]
    uint16_t *scl = (uint16_t *)(sb + MR * ncol * bs);  // [ncol][bs]
    float *wmax = FAST ? (float *)(xy + ncol * bs2) : (float *)(scl + ncol * bs);  // [MR][WV]
    int32_t *wsum = (int32_t *)(wmax + MR * WV);        // [MR][WV]

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int gq4 = lane >> 4, c = lane & 15;
    // wave -> (column group gi, K range kw): 8 / CG waves share a column group
    const uint32_t wpg_shift = 3 - cg_shift;
    const uint32_t gi = (uint32_t)wave >> wpg_shift, kw = (uint32_t)wave & ((1u << wpg_shift) - 1);
    const uint32_t wg_col0 = xcd_tile(blockIdx.x, tiles) * ncol;
    const uint32_t col0 = wg_col0 + gi * 16;  // this wave's 16 columns
    const rsrc_t ar = make_rsrc(src, m * k * 2u);
    const bool vec = (k & 7) == 0;

    // -- 1. loads: A or its quantized rows (waited on first), codes, scales
    uint4 areg[QP][MR];
    uint4 qreg[MR];
    float pqs[PQ];      // quantized rows' block scales and sums, entries t + T*j
    int32_t pqsum[PQ];  // (m * nbq <= PQ * T: the host checks)
    if constexpr (MR > 1) {
        const rsrc_t qr = make_rsrc(src, m * kq);
#pragma unroll
        for (int r = 0; r < MR; r++)
            qreg[r] = bload16(qr, ((uint32_t)r < m && 16u * t < kq) ? r * kq + 16 * t : OOB);
    } else {
#pragma unroll
        for (int p = 0; p < QP; p++)
#pragma unroll
            for (int r = 0; r < MR; r++)
                areg[p][r] = (uint32_t)p * QPASS < kq ? load_row8(ar, r, m, k, p * QPASS + 8 * t, vec)
                                                      : make_uint4(0, 0, 0, 0);
    }
    // scale rows next (waited on before the first barrier), then the codes,
    // then the epilogue operands: vmcnt retires in issue order, so the codes
    // can still be in flight when the waits before them end
    uint4 sreg = {};
    uint2 sreg4 = {};  // FAST: the scales of this lane's block and four columns
    const uint32_t fb = kw * NBW + (uint32_t)c;  // FAST: this lane's block (c < NBW)
    {
        const rsrc_t sr = make_rsrc(sc, ((sc_rows + 3) & ~3u) * n_pad * 2u);
        if constexpr (FAST) {
            sreg4 = bload8(sr, ((uint32_t)c < (uint32_t)NBW && fb < sc_rows)
                                   ? (uint32_t)cell_index(fb, col0 + 4 * gq4, sc_rows, n_pad) * 2u : OOB);
        } else {
            const uint32_t bb = t >> (cg_shift + 1), piece = t & (2 * cg - 1);  // 8 columns a piece
            sreg = bload16(sr, (bb < nbq && bb < sc_rows)
                                   ? (uint32_t)cell_index(bb, wg_col0 + piece * 8, sc_rows, n_pad) * 2u : OOB);
        }
    }
    uint4 wreg[NG];
    {
        const rsrc_t cr = make_rsrc(codes, ((ngroups + 3) & ~3u) * n_pad * 64u);
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const uint32_t grp = kw * NG + i;
            wreg[i] = bload16(cr, grp < ngroups ? ((uint32_t)cell_index(grp, col0 + c, ngroups, n_pad) * 4 + gq4) * 16 : OOB);
        }
    }
    // every code load is issued before anything below: the scalar loads of
    // the arguments past the preloaded ones (n, the epilogue's) must not be
    // hoisted between them, where their wait would hold the later code loads
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MR > 1) {
        // the rows' block scales and sums: their pointers are arguments past
        // the preloaded ones
        const float *qs = (const float *)((const uint8_t *)src + ((m * kq + 255) & ~255u));
        const int32_t *qsum = (const int32_t *)(qs + m * nbq);
        const rsrc_t fr = make_rsrc(qs, m * nbq * 4u), ur = make_rsrc(qsum, m * nbq * 4u);
#pragma unroll
        for (int j = 0; j < PQ; j++) {
            const uint32_t i = t + T * j;
            pqs[j] = __uint_as_float(bload4(fr, i < m * nbq ? i * 4u : OOB));
            pqsum[j] = (int32_t)bload4(ur, i < m * nbq ? i * 4u : OOB);
        }
    }
    // this lane's block-sum slot (step 3), computed before the epilogue loads
    // and pinned to a register of its own: the compiler can otherwise build it
    // late with a 64-bit multiply-add whose unused high half is a register
    // one of those loads targets, and wait for that load
    uint32_t dp_off = FAST ? 0u : (c * ncol + gi * 16 + 4 * gq4) * bs;
    if constexpr (!FAST) asm volatile("" : "+v"(dp_off));
    const bool folder = (uint32_t)t < ncol * m;
    const int fc = t & (ncol - 1), frow = t >> (4 + cg_shift);

    // -- 2. quantize A (quantize_row, src/kernels/lowbit/matmul.rs:354-371),
    //       or store the rows quantized beforehand
    if constexpr (MR > 1) {
#pragma unroll
        for (int r = 0; r < MR; r++)
            if (16u * t < kq) *(uint4 *)(ql + r * qs_ + 16 * t) = qreg[r];
#pragma unroll
        for (int j = 0; j < PQ; j++) {
            const uint32_t i = t + T * j;
            if (i < MR * nbq) {  // rows m..MR-1 read zeros
                sa[i] = pqs[j];
                as[i] = pqsum[j];
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < QP; p++) {
            if ((uint32_t)p * QPASS >= kq) break;  // uniform
            quant_pass<KIND, MR, SPB == 2 ? 7 : 0>(areg[p], p, ql, qs_, sa, as, nbq, kq, block_shift, wmax, wsum);
        }
    }
    // the epilogue operands after the quantization: their addresses wait on
    // scalar loads of kernel arguments, which must hold up neither the codes
    // nor the quantization (the operands are used only at the store)
    EpPre pre = {};
    uint16_t opa = 0, opb = 0;
    if constexpr (EPV == 0) {
        if (folder && wg_col0 + fc < n) pre = ep_prefetch(ep, frow, wg_col0 + fc, n);
    } else if constexpr (EPV >= 2) {
        const uint32_t ob = folder && wg_col0 + fc < n ? (wg_col0 + fc) * 2u : OOB;
        opb = bload2(make_rsrc(col_b, n * 2u), ob);
        if constexpr (EPV == 3) opa = bload2(make_rsrc(col_a, n * 2u), ob);
    }

    if constexpr (FAST) {
        if (t < 4) *(uint4 *)(ql + qs_ + 16 * t) = make_uint4(0, 0, 0, 0);  // the zero B operand
    } else if ((uint32_t)t < 2 * cg * nbq) {  // transpose: scale of (block bb, column 8 piece + e)
        const uint32_t bb = t >> (cg_shift + 1), piece = t & (2 * cg - 1);
        const uint32_t sw[4] = {sreg.x, sreg.y, sreg.z, sreg.w};
#pragma unroll
        for (int e = 0; e < 8; e++) scl[(8 * piece + e) * bs + bb] = (uint16_t)(sw[e / 2] >> (16 * (e % 2)));
    }
    __syncthreads();
    const uint32_t nb_live = (k + block - 1) >> block_shift;

    // -- 3. exact block sums on the matrix cores: A = 16 columns x 64 depths
    //       of expanded codes, B = 64 depths x up to 16 rows of q
    // lane (gq4, c) holds the sums of columns 4*gq4 + v, row c; rows m..MR-1
    // of q are zero, so their sums are too
    int32_t *dp = sb + dp_off;
    // (the q fragments below are not masked: lanes c >= MR read row 0 again,
    // and an MFMA's output column c depends only on its B column c, so those
    // lanes' sums are never stored)
    auto expand = [&](int i) {
        const uint4 wv = wreg[i / SPG];
        const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
        int4_t wa;
        if (KIND == 2) {
            const uint32_t w = words[i % 4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                wa[j] = (int)__builtin_amdgcn_perm(codebook, codebook, (w >> (2 * j)) & 0x03030303u);
        } else {
            const uint32_t w = words[(i % 8) / 2], hs = 4 * (i % 2);
#pragma unroll
            for (int j = 0; j < 4; j++) wa[j] = (int)((w >> (hs + j)) & 0x01010101u);
        }
        return wa;
    };
    // q fragments: every lane reads a valid row, unconditionally, so a
    // group's reads are issued together and overlap instead of each one
    // preceding its MFMA
    auto qload = [&](int i) {
        const uint32_t slab = kw * NSW + i;
        return __builtin_bit_cast(int4_t, *(const uint4 *)(ql + (c < MR ? c : 0) * qs_ + slab * LB_SLAB + 16 * gq4));
    };
    constexpr int PF = NSW < 8 ? NSW : 8;  // slabs whose q is read ahead at once
    if constexpr (FAST) {
        // B column c is q on block c's slabs (slab i belongs to block i / 2)
        // and zero elsewhere: one address select per slab
        auto qloadf = [&](int i) {
            const uint32_t slab = kw * NSW + i;
            const int8_t *pa = (c == i / SPB) ? ql + slab * LB_SLAB + 16 * gq4 : zq + 16 * gq4;
            return __builtin_bit_cast(int4_t, *(const uint4 *)pa);
        };
        int4_t acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};  // a block's first and second slab
#pragma unroll
        for (int i0 = 0; i0 < NSW; i0 += PF) {
            int4_t qv[PF];
#pragma unroll
            for (int j = 0; j < PF; j++) qv[j] = qloadf(i0 + j);
#pragma unroll
            for (int j = 0; j < PF; j++) {
                if ((i0 + j) % 2 == 0) acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(expand(i0 + j), qv[j], acc0, 0, 0, 0);
                else acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(expand(i0 + j), qv[j], acc1, 0, 0, 0);
            }
        }
        // lane (gq4, c < NBW): block fb's sums of columns 4 gq4 + v; its fold
        // factors x = f32(sum) (Q1: 2 sum(q b) + (-sum(q))) and y =
        // f32(scale) * s by v_fma_mix (the f16 scale widened exactly, one
        // rounding, the -0 addend leaves the product as it is); blocks past K
        // give x = y = 0
        if ((uint32_t)c < (uint32_t)NBW) {
            const float s_b = sa[fb];
            const int32_t a_b = KIND == 1 ? as[fb] : 0;
            const bool live = fb < nb_live;
            float2 *xo = xy + (gi * 16 + 4 * gq4) * bs2 + fb;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int32_t sum = acc0[v] + acc1[v];
                float x = (float)(KIND == 1 ? 2 * sum + a_b : sum), y;
                const uint32_t cw = v < 2 ? sreg4.x : sreg4.y;
                if (v % 2 == 0)
                    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(y) : "v"(cw), "v"(s_b), "v"(-0.0f));
                else
                    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                        : "=v"(y) : "v"(cw), "v"(s_b), "v"(-0.0f));
                if (!live) x = y = 0.0f;
                xo[v * bs2] = make_float2(x, y);
            }
        }
    } else if constexpr (SPB > 0) {
        // blocks of SPB slabs, whole inside this wave's range; independent
        // accumulators, written after the last product
        constexpr int NBW = NSW / SPB;
        int4_t acc[NBW];
#pragma unroll
        for (int b = 0; b < NBW; b++) acc[b] = (int4_t){0, 0, 0, 0};
#pragma unroll
        for (int i0 = 0; i0 < NSW; i0 += PF) {
            int4_t qv[PF];
#pragma unroll
            for (int j = 0; j < PF; j++) qv[j] = qload(i0 + j);
#pragma unroll
            for (int j = 0; j < PF; j++)
                acc[(i0 + j) / SPB] =
                    __builtin_amdgcn_mfma_i32_16x16x64_i8(expand(i0 + j), qv[j], acc[(i0 + j) / SPB], 0, 0, 0);
        }
        if constexpr (MR == 1) {
            // row 0's lanes (c = 0) store their four columns' sums of each
            // block at once: [block][column]
            if (c == 0) {
                int32_t *o = sb + kw * NBW * ncol + gi * 16 + 4 * gq4;
#pragma unroll
                for (int b = 0; b < NBW; b++) *(int4_t *)(o + b * ncol) = acc[b];
            }
        } else if (c < MR) {
            // block kw * NBW + b < kq / block <= nbq (the waves hold whole
            // blocks); one base offset per column, held in a register of its
            // own, and the block as the stores' immediate offset
            uint32_t o[4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                o[v] = dp_off + v * bs + kw * NBW;
                asm volatile("" : "+v"(o[v]));
            }
#pragma unroll
            for (int b = 0; b < NBW; b++)
#pragma unroll
                for (int v = 0; v < 4; v++) sb[o[v] + b] = acc[b][v];
        }
    } else {
        const uint32_t parts = block < (uint32_t)LB_SLAB ? LB_SLAB / block : 1;
        const uint32_t spb = block > (uint32_t)LB_SLAB ? block / LB_SLAB : 1;  // slabs per block
        int4_t acc = {0, 0, 0, 0};
        int4_t qv[PF];
#pragma unroll
        for (int i = 0; i < NSW; i++) {
            if (i % PF == 0) {
#pragma unroll
                for (int j = 0; j < PF; j++) qv[j] = qload(i + j);
            }
            const uint32_t slab = kw * NSW + i;
            const int4_t wa = expand(i), ab = qv[i % PF];
            if (parts == 1) {
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, ab, acc, 0, 0, 0);
                if ((slab + 1) % spb == 0) {  // uniform: the block ends in this wave
                    const uint32_t bb = slab / spb;
                    if (c < MR && bb < nbq) {
#pragma unroll
                        for (int v = 0; v < 4; v++) dp[v * bs + bb] = acc[v];
                    }
                    acc = (int4_t){0, 0, 0, 0};
                }
            } else {
                // blocks shorter than a slab: one masked product per block
                for (uint32_t pp = 0; pp < parts; pp++) {
                    const int4_t abp = (uint32_t)(16 * gq4) / block == pp ? ab : (int4_t){0, 0, 0, 0};
                    const int4_t r4 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, abp, (int4_t){0, 0, 0, 0}, 0, 0, 0);
                    const uint32_t bb = slab * parts + pp;
                    if (c < MR && bb < nbq) {
#pragma unroll
                        for (int v = 0; v < 4; v++) dp[v * bs + bb] = r4[v];
                    }
                }
            }
        }
    }
    __syncthreads();

    // -- 4. fold in block order (reference, matmul.rs:380-393): per block
    //       x = f32(sum) (Q1: 2*sum(q*b) + (-sum(q))) and y = f32(scale)*s by
    //       v_fma_mix (the f16 operand widened exactly, one rounding; the -0
    //       addend leaves every product as it is), then total = fmaf(x, y,
    //       total). Blocks past K add fmaf(0, 0, total) == total (total starts
    //       at +0 and never becomes -0, so its bits are unchanged).
    float total = 0.0f;
    if constexpr (FAST) {
        // (x, y) of blocks 0 .. nb_live - 1 in order, two blocks a 16-byte
        // load: whole groups of 16 blocks, then the last group's live pairs
        // (a wave's range is an even number of blocks, so a pair that starts
        // below nb_live was written)
        if (folder) {
            const float *xp = (const float *)(xy + fc * bs2);
            auto group16 = [&](uint32_t b0, auto tail_tag) {
                constexpr bool TAIL = decltype(tail_tag)::value;
                float4_t v4[8];
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    const bool live = !TAIL || b0 + 2 * h < nb_live;
                    v4[h] = *(const float4_t *)(xp + 2 * (live ? b0 + 2 * h : 0));
                    if (TAIL && !live) v4[h] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    total = fmaf(v4[h][0], v4[h][1], total);
                    total = fmaf(v4[h][2], v4[h][3], total);
                }
            };
            const uint32_t nb16 = nb_live & ~15u;
            for (uint32_t b0 = 0; b0 < nb16; b0 += 16) group16(b0, std::false_type{});
            if (nb16 < nb_live) group16(nb16, std::true_type{});
        }
    } else if constexpr (MR == 1) {
        // one row: 16 * CG folding lanes, so every thread first computes a
        // few blocks' x and y, and the folding lanes then only load them, 16
        // blocks per four LDS loads, and run the fmas
        const uint32_t nbf = (nb_live + 3) & ~3u;  // <= nbq; x = y = 0 past nb_live
        {
            const uint32_t j = t & (ncol - 1), bstep = (uint32_t)T >> (4 + cg_shift);
            for (uint32_t b = (uint32_t)t >> (4 + cg_shift); b < nbf; b += bstep) {
                const uint32_t e = j * bs + b;
                float x = 0.0f, y = 0.0f;
                if (b < nb_live) {
                    const int32_t sum = SPB > 0 ? sb[b * ncol + j] : sb[e];  // the products' layouts
                    x = (float)(KIND == 1 ? 2 * sum + as[b] : sum);
                    const uint32_t cw = scl[e];
                    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(y) : "v"(cw), "v"(sa[b]), "v"(-0.0f));
                }
                xl[e] = x;
                yl[e] = y;
            }
        }
        __syncthreads();
        if (folder) {
            const float *xp = xl + fc * bs;
            const float *yp = yl + fc * bs;
            auto group16 = [&](uint32_t b0, auto tail_tag) {
                constexpr bool TAIL = decltype(tail_tag)::value;
                float4_t x4[4], y4[4];
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const bool live = !TAIL || b0 + 4 * h < nbf;
                    const uint32_t bh = live ? b0 + 4 * h : 0;
                    x4[h] = *(const float4_t *)(xp + bh);
                    y4[h] = *(const float4_t *)(yp + bh);
                    if (TAIL && !live) x4[h] = y4[h] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int h = 0; h < 4; h++)
#pragma unroll
                    for (int u = 0; u < 4; u++) total = fmaf(x4[h][u], y4[h][u], total);
            };
            const uint32_t nb16 = nbf & ~15u;
            for (uint32_t b0 = 0; b0 < nb16; b0 += 16) group16(b0, std::false_type{});
            if (nb16 < nbf) group16(nb16, std::true_type{});
        }
    } else if (folder) {
        // several rows: 16 * CG lanes per row fold, each reading four blocks'
        // sums, scales and factors per LDS load
        const int32_t *sp = sb + (frow * ncol + fc) * bs;
        const uint16_t *cp = scl + fc * bs;
        const float *ap = sa + frow * nbq;
        const int32_t *qp = as + frow * nbq;
        // 16 blocks from b0; TAIL: some are past K, zeroed by selects
        auto group16 = [&](uint32_t b0, auto tail_tag) {
            constexpr bool TAIL = decltype(tail_tag)::value;
            int4_t s4[4], q4[4];
            uint2 c4[4];
            float4_t a4[4];
#pragma unroll
            for (int h = 0; h < 4; h++) {  // 16 blocks' operands in flight before the fma chain
                const uint32_t bh = !TAIL || b0 + 4 * h < nbq ? b0 + 4 * h : 0;
                s4[h] = *(const int4_t *)(sp + bh);
                c4[h] = *(const uint2 *)(cp + bh);
                a4[h] = *(const float4_t *)(ap + bh);
                q4[h] = KIND == 1 ? *(const int4_t *)(qp + bh) : (int4_t){0, 0, 0, 0};
            }
#pragma unroll
            for (int h = 0; h < 4; h++) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int32_t sum = KIND == 1 ? 2 * s4[h][u] + q4[h][u] : s4[h][u];
                    const uint32_t cw = u < 2 ? c4[h].x : c4[h].y;
                    float y;
                    if (u % 2 == 0)
                        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]"
                            : "=v"(y) : "v"(cw), "v"(a4[h][u]), "v"(-0.0f));
                    else
                        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                            : "=v"(y) : "v"(cw), "v"(a4[h][u]), "v"(-0.0f));
                    float x = (float)sum;
                    if constexpr (TAIL) {
                        const bool live = b0 + 4 * h + u < nb_live;
                        x = live ? x : 0.0f;
                        y = live ? y : 0.0f;
                    }
                    total = fmaf(x, y, total);
                }
            }
        };
        const uint32_t nb_full = nb_live & ~15u;
        for (uint32_t b0 = 0; b0 < nb_full; b0 += 16) group16(b0, std::false_type{});
        if (nb_full < nb_live) group16(nb_full, std::true_type{});
    }
    if (folder) {
        const uint32_t j = wg_col0 + fc;
        if (j < n) {
            uint16_t out;
            if constexpr (EPV == 0) {
                out = finish_pre<false>(ep, pre, total, frow, j, n);
            } else {
                out = f32_to_f16(total);
                if constexpr (EPV >= 2) {
                    float x = f16_to_f32(out);
                    if constexpr (EPV == 3) x = x * f16_to_f32(opa);
                    x = x + f16_to_f32(opb);
                    out = act == EP_ACT_NONE ? f32_to_f16(x) : act_round16<false>(act, x, alpha);
                }
            }
            dst[(size_t)frow * n + j] = out;
        }
    }
}


// ---------------------------------------------------------------------------
// Up to 8 rows, blocks of 128 (the usual decode call), persistent: one
// workgroup per compute unit (grid G = min(tiles, CUs)), workgroup g taking
// tiles g, g + G, ... (up to TPW of them). Two workgroups on one compute unit
// were measured to serialize: the second one's activation loads queue behind
// the first one's weight stream, so it quantizes ~1.2 us later. Here a
// compute unit issues A first, then every tile's scales and codes, quantizes
// A once (every row: no separate quantization launch) and multiplies its
// tiles as their codes land:
//   1. loads: A (f16, one 4096-depth pass per thread and row), then per tile
//      the scales and code groups;
//   2. quant_pass into LDS (shared by the tiles), one barrier;
//   3. per tile, exact block sums on v_mfma_i32_16x16x64_i8. One row: block
//      c of the wave's range lands in output row c (the B operand's column c
//      holds q on that block's slabs, zero elsewhere), so the lanes holding a
//      block's sums form its fold factors x = f32(sum) (Q1: 2 sum(q b) +
//      (-sum(q))) and y = f32(scale) * s with scales they loaded themselves.
//      Several rows: B column c is row c; each block's sums accumulate over
//      its two slabs and x goes to LDS, the scales through an LDS transpose;
//   4. one barrier, then one thread per (tile, row, column) folds its blocks
//      in order (fmaf), runs the op-graph and stores.
// misc = cg_shift | act << 8 | m << 16. LDS (row_lds_bytes): q [MR][kq + 16]
// i8 | 64 zero bytes | s [MR][nbq] f32 | -sum(q) [MR][nbq] i32 | one row: (x,
// y) [TPW][16 CG][nbq + 2]; several: x [TPW][MR][16 CG][nbq + 4] f32 and
// scales [TPW][16 CG][nbq + 4] f16 | wave partials.
// ---------------------------------------------------------------------------
size_t row_lds_bytes(uint32_t kq, uint32_t nbq, uint32_t cg, int tpw, int mr) {
    const size_t head = (size_t)mr * (kq + 16) + 64 + (size_t)mr * nbq * 8;
    const size_t body = mr == 1 ? (size_t)tpw * 16 * cg * (nbq + 2) * 8
                                : (size_t)tpw * 16 * cg * (nbq + 4) * ((size_t)mr * 4 + 2);
    return head + body + (size_t)mr * WV * 8;
}

template <int KIND, int MR, int NG, int EPV, int TPW>
__global__ void __launch_bounds__(T)
    lowbit_row(const uint8_t *codes, const uint16_t *sc, const uint16_t *lhs, uint16_t *dst, const uint16_t *col_b,
               uint32_t k, uint32_t misc, uint32_t n, uint32_t codebook, const uint16_t *col_a, float alpha,
               EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr uint32_t SPG = KIND == 2 ? 4 : 8;  // slabs per code group
    constexpr int NSW = NG * (int)SPG;            // slabs per wave
    constexpr int NBW = NSW / 2;                  // blocks of 128 per wave
    static_assert(NBW >= 1 && NBW <= 16, "a wave's blocks are rows of one product tile");
    constexpr int QP = 2;                         // A passes held in registers (K <= 8192)
    constexpr uint32_t BSH = 7, BLOCK = 128;
    const uint32_t cg_shift = misc & 0xFF, act = (misc >> 8) & 0xFF, m = MR == 1 ? 1u : misc >> 16;
    const uint32_t n_pad = ((n ? n : 1u) + 127u) & ~127u;
    const uint32_t tiles = n_pad >> (4 + cg_shift);
    const uint32_t G = gridDim.x;
    const uint32_t kq = (8u >> cg_shift) * NSW * LB_SLAB;
    const uint32_t nbq = ((kq >> BSH) + 3) & ~3u;
    const uint32_t grp_depths = KIND == 2 ? Q2_GROUP : Q1_GROUP;
    const uint32_t ngroups = (k + grp_depths - 1) / grp_depths;
    const uint32_t sc_rows = (ngroups * grp_depths + BLOCK - 1) >> BSH;
    const uint32_t ncol = 16u << cg_shift;
    const uint32_t qs_ = kq + 16;
    const uint32_t bs = nbq + 4;   // several rows: x / scale row stride
    const uint32_t bs2 = nbq + 2;  // one row: (x, y) pair row stride
    int8_t *ql = (int8_t *)smem;                     // [MR][qs_]
    const int8_t *zq = ql + MR * qs_;                // 64 zero bytes
    float *sa = (float *)(smem + MR * qs_ + 64);     // [MR][nbq]
    int32_t *as = (int32_t *)(sa + MR * nbq);        // [MR][nbq]
    float2 *xy = (float2 *)(as + MR * nbq);          // one row: [TPW][ncol][bs2]
    float *xs = (float *)(as + MR * nbq);            // several: [TPW][MR][ncol][bs]
    uint16_t *scl = (uint16_t *)(xs + TPW * MR * ncol * bs);  // several: [TPW][ncol][bs]
    float *wmax = MR == 1 ? (float *)(xy + TPW * ncol * bs2) : (float *)(scl + TPW * ncol * bs);
    int32_t *wsum = (int32_t *)(wmax + MR * WV);

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int gq4 = lane >> 4, c = lane & 15;
    const uint32_t wpg_shift = 3 - cg_shift;
    const uint32_t gi = (uint32_t)wave >> wpg_shift, kw = (uint32_t)wave & ((1u << wpg_shift) - 1);
    const uint32_t fb = kw * NBW + (uint32_t)c;  // one row: this lane's block (c < NBW)

    // -- 1. loads: A, then each tile's scales and codes
    uint4 areg[QP][MR];
    {
        const rsrc_t ar = make_rsrc(lhs, m * k * 2u);
        const bool vec = (k & 7) == 0;
#pragma unroll
        for (int p = 0; p < QP; p++)
#pragma unroll
            for (int r = 0; r < MR; r++)
                areg[p][r] = (uint32_t)p * QPASS < kq ? load_row8(ar, r, m, k, p * QPASS + 8 * t, vec)
                                                      : make_uint4(0, 0, 0, 0);
    }
    bool tlive[TPW];
    uint2 sreg4[TPW];  // one row: the lane's block, four columns
    uint4 sreg[TPW];   // several rows: block t / (2 CG), eight columns
    uint4 wreg[TPW][NG];
    {
        const rsrc_t sr = make_rsrc(sc, ((sc_rows + 3) & ~3u) * n_pad * 2u);
        const rsrc_t cr = make_rsrc(codes, ((ngroups + 3) & ~3u) * n_pad * 64u);
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const uint32_t li = blockIdx.x + j * G;
            tlive[j] = li < tiles;
            const uint32_t tcol0 = xcd_tile(tlive[j] ? li : 0, tiles) * ncol;
            const uint32_t col0 = tcol0 + gi * 16;
            if constexpr (MR == 1) {
                sreg4[j] = bload8(sr, (tlive[j] && (uint32_t)c < (uint32_t)NBW && fb < sc_rows)
                                          ? (uint32_t)cell_index(fb, col0 + 4 * gq4, sc_rows, n_pad) * 2u : OOB);
            } else {
                const uint32_t bb = t >> (cg_shift + 1), piece = t & (2 * (1u << cg_shift) - 1);
                sreg[j] = bload16(sr, (tlive[j] && bb < nbq && bb < sc_rows)
                                          ? (uint32_t)cell_index(bb, tcol0 + piece * 8, sc_rows, n_pad) * 2u : OOB);
            }
#pragma unroll
            for (int i = 0; i < NG; i++) {
                const uint32_t grp = kw * NG + i;
                wreg[j][i] = bload16(cr, tlive[j] && grp < ngroups
                                             ? ((uint32_t)cell_index(grp, col0 + c, ngroups, n_pad) * 4 + gq4) * 16 : OOB);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // -- 2. quantize A once for every tile of this workgroup
#pragma unroll
    for (int p = 0; p < QP; p++) {
        if ((uint32_t)p * QPASS >= kq) break;  // uniform
        quant_pass<KIND, MR, BSH>(areg[p], p, ql, qs_, sa, as, nbq, kq, BSH, wmax, wsum);
    }
    // the epilogue operands of the (tile, row, column) this thread folds
    const uint32_t fj = (uint32_t)t / (MR * ncol), frow = ((uint32_t)t / ncol) % MR, fc = (uint32_t)t & (ncol - 1);
    const bool folder = fj < (uint32_t)TPW && blockIdx.x + fj * G < tiles && frow < m;
    const uint32_t fcol = (folder ? xcd_tile(blockIdx.x + fj * G, tiles) * ncol : 0) + fc;
    EpPre pre = {};
    uint16_t opa = 0, opb = 0;
    if constexpr (EPV == 0) {
        if (folder && fcol < n) pre = ep_prefetch(ep, frow, fcol, n);
    } else if constexpr (EPV >= 2) {
        const uint32_t ob = folder && fcol < n ? fcol * 2u : OOB;
        opb = bload2(make_rsrc(col_b, n * 2u), ob);
        if constexpr (EPV == 3) opa = bload2(make_rsrc(col_a, n * 2u), ob);
    }
    if (t < 4) *(uint4 *)(ql + MR * qs_ + 16 * t) = make_uint4(0, 0, 0, 0);  // the zero B operand
    __syncthreads();
    const uint32_t nb_live = (k + BLOCK - 1) >> BSH;

    // -- 3. per tile: exact block sums, then the fold factors
    const float s_b = MR == 1 && (uint32_t)c < (uint32_t)NBW ? sa[fb] : 0.0f;
    const int32_t a_b = MR == 1 && KIND == 1 && (uint32_t)c < (uint32_t)NBW ? as[fb] : 0;
    constexpr int PF = NSW < 8 ? NSW : 8;
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        if (!tlive[j]) break;  // uniform; later tiles are past the last too
        auto expand = [&](int i) {
            const uint4 wv = wreg[j][i / SPG];
            const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
            int4_t wa;
            if (KIND == 2) {
                const uint32_t w = words[i % 4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    wa[e] = (int)__builtin_amdgcn_perm(codebook, codebook, (w >> (2 * e)) & 0x03030303u);
            } else {
                const uint32_t w = words[(i % 8) / 2], hs = 4 * (i % 2);
#pragma unroll
                for (int e = 0; e < 4; e++) wa[e] = (int)((w >> (hs + e)) & 0x01010101u);
            }
            return wa;
        };
        if constexpr (MR == 1) {
            auto qloadf = [&](int i) {
                const uint32_t slab = kw * NSW + i;
                const int8_t *pa = (c == i / 2) ? ql + slab * LB_SLAB + 16 * gq4 : zq + 16 * gq4;
                return __builtin_bit_cast(int4_t, *(const uint4 *)pa);
            };
            int4_t acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};  // a block's first and second slab
#pragma unroll
            for (int i0 = 0; i0 < NSW; i0 += PF) {
                int4_t qv[PF];
#pragma unroll
                for (int i = 0; i < PF; i++) qv[i] = qloadf(i0 + i);
#pragma unroll
                for (int i = 0; i < PF; i++) {
                    if ((i0 + i) % 2 == 0) acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(expand(i0 + i), qv[i], acc0, 0, 0, 0);
                    else acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(expand(i0 + i), qv[i], acc1, 0, 0, 0);
                }
            }
            if ((uint32_t)c < (uint32_t)NBW) {
                const bool live = fb < nb_live;
                float2 *xo = xy + ((uint32_t)j * ncol + gi * 16 + 4 * gq4) * bs2 + fb;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int32_t sum = acc0[v] + acc1[v];
                    float x = (float)(KIND == 1 ? 2 * sum + a_b : sum), y;
                    const uint32_t cw = v < 2 ? sreg4[j].x : sreg4[j].y;
                    if (v % 2 == 0)
                        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(y) : "v"(cw), "v"(s_b), "v"(-0.0f));
                    else
                        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                            : "=v"(y) : "v"(cw), "v"(s_b), "v"(-0.0f));
                    if (!live) x = y = 0.0f;
                    xo[v * bs2] = make_float2(x, y);
                }
            }
        } else {
            // B column c is row c (lanes c >= MR read row 0 again: their
            // output rows are never stored); block b's sums in acc[b]
            auto qload = [&](int i) {
                const uint32_t slab = kw * NSW + i;
                return __builtin_bit_cast(int4_t, *(const uint4 *)(ql + (c < MR ? c : 0) * qs_ + slab * LB_SLAB + 16 * gq4));
            };
            int4_t acc[NBW];
#pragma unroll
            for (int b = 0; b < NBW; b++) acc[b] = (int4_t){0, 0, 0, 0};
#pragma unroll
            for (int i0 = 0; i0 < NSW; i0 += PF) {
                int4_t qv[PF];
#pragma unroll
                for (int i = 0; i < PF; i++) qv[i] = qload(i0 + i);
#pragma unroll
                for (int i = 0; i < PF; i++)
                    acc[(i0 + i) / 2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(expand(i0 + i), qv[i], acc[(i0 + i) / 2], 0, 0, 0);
            }
            // x = f32(sum) (Q1: 2 sum + (-sum(q))) of row c, columns 4 gq4 + v,
            // this wave's blocks, four blocks a 16-byte store
            if (c < MR) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float *xo = xs + (((uint32_t)j * MR + c) * ncol + gi * 16 + 4 * gq4 + v) * bs + kw * NBW;
#pragma unroll
                    for (int b4 = 0; b4 < NBW; b4 += 4) {
                        float4_t x4;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const int b = b4 + e;
                            if (b < NBW) {
                                const int32_t sum = acc[b][v];
                                x4[e] = (float)(KIND == 1 ? 2 * sum + as[c * nbq + kw * NBW + b] : sum);
                            } else {
                                x4[e] = 0.0f;
                            }
                        }
                        if (b4 + 4 <= NBW) *(float4_t *)(xo + b4) = x4;
                        else
#pragma unroll
                            for (int e = 0; e < 4; e++)
                                if (b4 + e < NBW) xo[b4 + e] = x4[e];
                    }
                }
            }
            // the tile's scales, transposed: scale of (block bb, column 8 piece + e)
            if ((uint32_t)t < 2 * (1u << cg_shift) * nbq) {
                const uint32_t bb = t >> (cg_shift + 1), piece = t & (2 * (1u << cg_shift) - 1);
                const uint32_t sw[4] = {sreg[j].x, sreg[j].y, sreg[j].z, sreg[j].w};
                uint16_t *sp = scl + (uint32_t)j * ncol * bs;
#pragma unroll
                for (int e = 0; e < 8; e++) sp[(8 * piece + e) * bs + bb] = (uint16_t)(sw[e / 2] >> (16 * (e % 2)));
            }
        }
    }
    __syncthreads();

    // -- 4. fold in block order (reference, matmul.rs:380-393)
    if (folder) {
        float total = 0.0f;
        if constexpr (MR == 1) {
            // two blocks a 16-byte load: whole groups of 16 blocks, then the
            // last group's live pairs (a wave's range is an even number of
            // blocks, so a pair that starts below nb_live was written)
            const float *xp = (const float *)(xy + (fj * ncol + fc) * bs2);
            auto group16 = [&](uint32_t b0, auto tail_tag) {
                constexpr bool TAIL = decltype(tail_tag)::value;
                float4_t v4[8];
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    const bool live = !TAIL || b0 + 2 * h < nb_live;
                    v4[h] = *(const float4_t *)(xp + 2 * (live ? b0 + 2 * h : 0));
                    if (TAIL && !live) v4[h] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    total = fmaf(v4[h][0], v4[h][1], total);
                    total = fmaf(v4[h][2], v4[h][3], total);
                }
            };
            const uint32_t nb16 = nb_live & ~15u;
            for (uint32_t b0 = 0; b0 < nb16; b0 += 16) group16(b0, std::false_type{});
            if (nb16 < nb_live) group16(nb16, std::true_type{});
        } else {
            // per block: x, and y = f32(scale) * s by v_fma_mix (the f16 scale
            // widened exactly, one rounding); blocks past K add nothing
            const float *xp = xs + ((fj * MR + frow) * ncol + fc) * bs;
            const uint16_t *cp = scl + (fj * ncol + fc) * bs;
            const float *ap = sa + frow * nbq;
            auto group16 = [&](uint32_t b0, auto tail_tag) {
                constexpr bool TAIL = decltype(tail_tag)::value;
                float4_t x4[4], a4[4];
                uint2 c4[4];
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const uint32_t bh = !TAIL || b0 + 4 * h < nb_live ? b0 + 4 * h : 0;
                    x4[h] = *(const float4_t *)(xp + bh);
                    c4[h] = *(const uint2 *)(cp + bh);
                    a4[h] = *(const float4_t *)(ap + bh);
                }
#pragma unroll
                for (int h = 0; h < 4; h++) {
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const uint32_t cw = u < 2 ? c4[h].x : c4[h].y;
                        float y, x = x4[h][u];
                        if (u % 2 == 0)
                            asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]"
                                : "=v"(y) : "v"(cw), "v"(a4[h][u]), "v"(-0.0f));
                        else
                            asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                                : "=v"(y) : "v"(cw), "v"(a4[h][u]), "v"(-0.0f));
                        if constexpr (TAIL) {
                            const bool live = b0 + 4 * h + u < nb_live;
                            x = live ? x : 0.0f;
                            y = live ? y : 0.0f;
                        }
                        total = fmaf(x, y, total);
                    }
                }
            };
            const uint32_t nb_full = nb_live & ~15u;
            for (uint32_t b0 = 0; b0 < nb_full; b0 += 16) group16(b0, std::false_type{});
            if (nb_full < nb_live) group16(nb_full, std::true_type{});
        }
        if (fcol < n) {
            uint16_t out;
            if constexpr (EPV == 0) {
                out = finish_pre<false>(ep, pre, total, frow, fcol, n);
            } else {
                out = f32_to_f16(total);
                if constexpr (EPV >= 2) {
                    float x = f16_to_f32(out);
                    if constexpr (EPV == 3) x = x * f16_to_f32(opa);
                    x = x + f16_to_f32(opb);
                    out = act == EP_ACT_NONE ? f32_to_f16(x) : act_round16<false>(act, x, alpha);
                }
            }
            dst[(size_t)frow * n + fcol] = out;
        }
    }
}

template <int KIND, int MR, int NG, int SPB, int EPV>
hipError_t launch_tile_v(const LtArgs &g, const EpArgs &ep, const EpPick &pk, hipStream_t s) {
    const size_t lds = tile_lds_bytes(g.kq, g.nbq, MR, 1u << g.cg_shift, MR == 1 && SPB == 2);
    if (lds > 64 * 1024) {
        static bool attr = false;  // benign race: every setter writes the same value
        if (!attr) {
            const hipError_t e = hipFuncSetAttribute((const void *)lowbit_tile<KIND, MR, NG, SPB, EPV>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     160 * 1024);
            if (e != hipSuccess) return e;
            attr = true;
        }
    }
    const uint32_t tiles = g.n_pad / (16u << g.cg_shift);
    const void *src = MR > 1 ? (const void *)g.q : (const void *)g.lhs;
    // the kernel derives these from its other arguments
    const uint32_t grp = KIND == 2 ? Q2_GROUP : Q1_GROUP;
    if (g.n_pad != (((g.n ? g.n : 1u) + 127u) & ~127u) || g.ngroups != (g.k + grp - 1) / grp || pk.act > 0xFF ||
        (MR > 1 && ((const uint8_t *)g.qs != (const uint8_t *)g.q + ((g.m * g.kq + 255) & ~255u) ||
                    g.qsum != (const int32_t *)(g.qs + g.m * g.nbq))))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((lowbit_tile<KIND, MR, NG, SPB, EPV>), dim3(tiles), dim3(T), lds, s, g.codes, g.sc, src,
                       g.dst, pk.b, g.k, g.m | (g.block_shift << 8) | (g.cg_shift << 16) | (pk.act << 24), g.n,
                       g.codebook, pk.a, pk.alpha, ep);
    return hipGetLastError();
}

// Compiled stores serve the usual decode format (block 128, SPB 2); other
// blocks take the generic store.
template <int KIND, int MR, int NG, int SPB>
hipError_t launch_tile_t(const LtArgs &g, const EpArgs &ep, hipStream_t s) {
    const EpPick pk = SPB == 2 ? pick_ep(ep) : EpPick{0, nullptr, nullptr, EP_ACT_NONE, 0.0f};
    if constexpr (SPB == 2) {
        if (pk.v == 1) return launch_tile_v<KIND, MR, NG, SPB, 1>(g, ep, pk, s);
        if (pk.v == 2) return launch_tile_v<KIND, MR, NG, SPB, 2>(g, ep, pk, s);
        if (pk.v == 3) return launch_tile_v<KIND, MR, NG, SPB, 3>(g, ep, pk, s);
    }
    return launch_tile_v<KIND, MR, NG, SPB, 0>(g, ep, pk, s);
}

template <int KIND, int MR>
hipError_t launch_tile_ng(const LtArgs &g, const EpArgs &ep, int ng, hipStream_t s) {
    const bool b128 = g.block_shift == 7;
    if (ng <= 1) return b128 ? launch_tile_t<KIND, MR, 1, 2>(g, ep, s) : launch_tile_t<KIND, MR, 1, 0>(g, ep, s);
    if (ng <= 2) return b128 ? launch_tile_t<KIND, MR, 2, 2>(g, ep, s) : launch_tile_t<KIND, MR, 2, 0>(g, ep, s);
    if (ng <= 4 || KIND == 1)
        return b128 ? launch_tile_t<KIND, MR, 4, 2>(g, ep, s) : launch_tile_t<KIND, MR, 4, 0>(g, ep, s);
    constexpr int NG8 = KIND == 1 ? 4 : 8;
    return b128 ? launch_tile_t<KIND, MR, NG8, 2>(g, ep, s) : launch_tile_t<KIND, MR, NG8, 0>(g, ep, s);
}

template <int KIND>
hipError_t launch_tile(const LtArgs &g, const EpArgs &ep, int mr, int ng, hipStream_t s) {
    if (mr <= 1) return launch_tile_ng<KIND, 1>(g, ep, ng, s);
    if (mr <= 2) return launch_tile_ng<KIND, 2>(g, ep, ng, s);
    if (mr <= 4) return launch_tile_ng<KIND, 4>(g, ep, ng, s);
    return launch_tile_ng<KIND, 8>(g, ep, ng, s);
}


// The persistent kernel (lowbit_row): up to 8 rows, blocks of 128, compiled
// stores only (the interpreted graph, Q2 with 8 code groups a lane, more than
// 4 tiles a compute unit and LDS past 150 KB take lowbit_tile);
// hipErrorNotSupported leaves those to it.
template <int KIND, int MR, int NG, int EPV, int TPW>
hipError_t launch_row_v(const LtArgs &g, const EpArgs &ep, const EpPick &pk, uint32_t grid, hipStream_t s) {
    const size_t lds = row_lds_bytes(g.kq, g.nbq, 1u << g.cg_shift, TPW, MR);
    if (lds > 64 * 1024) {
        static bool attr = false;  // benign race: every setter writes the same value
        if (!attr) {
            const hipError_t e = hipFuncSetAttribute((const void *)lowbit_row<KIND, MR, NG, EPV, TPW>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            if (e != hipSuccess) return e;
            attr = true;
        }
    }
    hipLaunchKernelGGL((lowbit_row<KIND, MR, NG, EPV, TPW>), dim3(grid), dim3(T), lds, s, g.codes, g.sc, g.lhs,
                       g.dst, pk.b, g.k, g.cg_shift | (pk.act << 8) | (g.m << 16), g.n, g.codebook, pk.a, pk.alpha,
                       ep);
    return hipGetLastError();
}
template <int KIND, int MR, int NG, int EPV>
hipError_t launch_row_t(const LtArgs &g, const EpArgs &ep, const EpPick &pk, uint32_t grid, int tpw, hipStream_t s) {
    switch (tpw) {
    case 1: return launch_row_v<KIND, MR, NG, EPV, 1>(g, ep, pk, grid, s);
    case 2: return launch_row_v<KIND, MR, NG, EPV, 2>(g, ep, pk, grid, s);
    case 3: return launch_row_v<KIND, MR, NG, EPV, 3>(g, ep, pk, grid, s);
    default: return launch_row_v<KIND, MR, NG, EPV, 4>(g, ep, pk, grid, s);
    }
}
template <int KIND, int MR, int NG>
hipError_t launch_row_e(const LtArgs &g, const EpArgs &ep, uint32_t grid, int tpw, hipStream_t s) {
    const EpPick pk = pick_ep(ep);
    if (pk.act > 0xFF) return hipErrorNotSupported;
    if (pk.v == 1) return launch_row_t<KIND, MR, NG, 1>(g, ep, pk, grid, tpw, s);
    if (pk.v == 2) return launch_row_t<KIND, MR, NG, 2>(g, ep, pk, grid, tpw, s);
    if (pk.v == 3) return launch_row_t<KIND, MR, NG, 3>(g, ep, pk, grid, tpw, s);
    return hipErrorNotSupported;
}
template <int KIND, int MR>
hipError_t launch_row_ng(const LtArgs &g, const EpArgs &ep, int ng, uint32_t grid, int tpw, hipStream_t s) {
    if (ng <= 1) return launch_row_e<KIND, MR, 1>(g, ep, grid, tpw, s);
    if (ng <= 2) return launch_row_e<KIND, MR, 2>(g, ep, grid, tpw, s);
    if (ng <= 4) return launch_row_e<KIND, MR, 4>(g, ep, grid, tpw, s);
    return hipErrorNotSupported;
}
// The persistent grid's shape for a call of tile_geometry sg: its workgroups
// and tiles a workgroup, or tpw = 0 when lowbit_row does not serve the call.
struct RowShape {
    uint32_t grid;
    int tpw;
};
template <int KIND>
hipError_t launch_row(const LtArgs &g, const EpArgs &ep, int ng, const RowShape &rs, hipStream_t s) {
    const uint32_t grid = rs.grid;
    const int tpw = rs.tpw;
    const int mr = g.m <= 1 ? 1 : g.m <= 2 ? 2 : g.m <= 4 ? 4 : 8;
    if (tpw < 1) return hipErrorNotSupported;
    if (mr == 1) return launch_row_ng<KIND, 1>(g, ep, ng, grid, tpw, s);
    if (mr == 2) return launch_row_ng<KIND, 2>(g, ep, ng, grid, tpw, s);
    if (mr == 4) return launch_row_ng<KIND, 4>(g, ep, ng, grid, tpw, s);
    return launch_row_ng<KIND, 8>(g, ep, ng, grid, tpw, s);
}

// One workgroup per (row, block): q for the block's depths (zero past k), the
// block's s = amax/127 and sum(q). Blocks from k up to kq are all zero.
__global__ void __launch_bounds__(256) lowbit_quant(const uint16_t *lhs, uint32_t k,
                                                    uint32_t block, uint32_t nbq, int8_t *q,
                                                    float *s, int32_t *asum, uint32_t kq) {
    __shared__ float red[256];
    __shared__ int redn[256];
    const uint32_t b = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    const uint32_t d0 = b * block, d1 = min(d0 + block, k);
    const uint16_t *src = lhs + (size_t)r * k;
    float amax = 0.0f;
    int nan = 0;
    for (uint32_t d = d0 + t; d < d1; d += 256) {
        const float x = fabsf(f16_to_f32(src[d]));
        if (x != x) nan = 1;
        amax = fmaxf(amax, x);
    }
    red[t] = amax;
    redn[t] = nan;
    __syncthreads();
    for (uint32_t off = 128; off > 0; off >>= 1) {
        if (t < off) {
            red[t] = fmaxf(red[t], red[t + off]);
            redn[t] |= redn[t + off];
        }
        __syncthreads();
    }
    amax = redn[0] ? __builtin_nanf("") : red[0];
    __syncthreads();
    const float inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    int qs = 0;
    for (uint32_t d = d0 + t; d < d0 + block && d < kq; d += 256) {
        int qi = 0;
        if (d < d1) {
            const float v = rintf(f16_to_f32(src[d]) * inv);
            qi = (v != v) ? 0 : (int)fminf(fmaxf(v, -128.0f), 127.0f);
        }
        q[(size_t)r * kq + d] = (int8_t)qi;
        qs += qi;
    }
    redn[t] = qs;
    __syncthreads();
    for (uint32_t off = 128; off > 0; off >>= 1) {
        if (t < off) redn[t] += redn[t + off];
        __syncthreads();
    }
    if (t == 0) {
        s[(size_t)r * nbq + b] = __fdiv_rn(amax, 127.0f);
        asum[(size_t)r * nbq + b] = redn[0];
    }
}

inline uint32_t ilog2(size_t x) { return (uint32_t)(63 - __builtin_clzll(x)); }
inline int rows_per_group(size_t m) {
    return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16;
}

// Geometry shared by the scratch sizing and the launch.
struct Geo {
    size_t unit, kq, nbq, seg;
};
Geo geometry(const WDev &w, size_t m) {
    Geo ge;
    ge.unit = w.block > (size_t)LB_SLAB ? w.block : (size_t)LB_SLAB;
    ge.kq = (w.k + ge.unit - 1) / ge.unit * ge.unit;
    if (ge.kq == 0) ge.kq = ge.unit;
    ge.nbq = ge.kq / w.block;
    const int mr = rows_per_group(m);
    // a segment: at most MAXS slabs per wave; its block sums fit S_BUDGET and
    // its block scales the staging registers (blocks may be longer than it)
    size_t seg = (size_t)WV * MAXS * LB_SLAB;
    while (seg > (size_t)LB_SLAB && (seg / w.block) * 16 * mr * 4 > (size_t)S_BUDGET) seg /= 2;
    while (seg > (size_t)LB_SLAB && seg / w.block > 2 * (size_t)T / mr) seg /= 2;
    ge.seg = seg;
    return ge;
}

template <int KIND, int MR>
hipError_t launch_t(const LbArgs &g, const EpArgs &ep, hipStream_t s) {
    const size_t nbs = g.seg_depths >= (1u << g.block_shift) ? (size_t)g.seg_depths >> g.block_shift : 1;
    const size_t lds = nbs * 16 * MR * 4 + nbs * 16 * 2 + 2 * MR * nbs * 4;
    static bool attr = false;  // benign race: every setter writes the same value
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)lowbit_gemv<KIND, MR>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 160 * 1024);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const dim3 grid((unsigned)(g.n_pad / 16), (unsigned)((g.m + MR - 1) / MR));
    hipLaunchKernelGGL((lowbit_gemv<KIND, MR>), grid, dim3(T), lds, s, g, ep);
    return hipGetLastError();
}

template <int KIND>
hipError_t launch_kind(const LbArgs &g, const EpArgs &ep, int mr, hipStream_t s) {
    if (mr <= 1) return launch_t<KIND, 1>(g, ep, s);
    if (mr <= 2) return launch_t<KIND, 2>(g, ep, s);
    if (mr <= 4) return launch_t<KIND, 4>(g, ep, s);
    if (mr <= 8) return launch_t<KIND, 8>(g, ep, s);
    return launch_t<KIND, 16>(g, ep, s);
}

// The single-launch path's geometry: code groups per lane (NG), the depths
// the waves cover and the blocks in them; it serves the decode shapes (up to
// 8 rows, blocks up to one quantization pass, K up to 8192, A in LDS).
struct TileGeo {
    bool ok;
    int ng;
    uint32_t kq, nbq, cg_shift;
};
// Column groups per workgroup (CG): enough that the grid stays within a few
// workgroups per CU (the per-workgroup staging of A and the fold are then paid
// a few times per CU); a wave's K range grows with them.
TileGeo tile_geometry_cg(const WDev &w, size_t m, uint32_t cg_shift) {
    TileGeo sg = {false, 0, 0, 0, cg_shift};
    const int mr = m <= 2 ? (int)m : m <= 4 ? 4 : 8;  // the row counts the kernel is built for
    const size_t spg = w.kind == W_Q2 ? 4 : 8;
    const size_t wpg = (size_t)WV >> cg_shift;   // waves along K per column group
    const size_t nslab = (w.k + LB_SLAB - 1) / LB_SLAB;
    const size_t per_wave = (nslab + wpg - 1) / wpg;
    const size_t ng_need = (per_wave + spg - 1) / spg;
    const size_t ng_max = w.kind == W_Q2 ? 8 : 4;
    if (ng_need > ng_max) return sg;
    const int ng = ng_need <= 1 ? 1 : ng_need <= 2 ? 2 : ng_need <= 4 ? 4 : 8;
    const size_t kq = wpg * ng * spg * LB_SLAB;
    if (kq > 2 * QPASS || kq < w.block || (size_t)mr * kq > 32768) return sg;
    // a wave's K range must hold whole blocks (block sums stay in one wave)
    if (w.block > (size_t)ng * spg * LB_SLAB) return sg;
    const size_t nbq = (kq / w.block + 3) / 4 * 4;  // whole 16-byte runs of blocks
    const size_t cg = (size_t)1 << cg_shift;
    if (2 * cg * nbq > (size_t)T || tile_lds_bytes((uint32_t)kq, (uint32_t)nbq, mr, (uint32_t)cg, mr == 1 && w.block == 128) > 96 * 1024)
        return sg;
    if (mr > 1 && (size_t)mr * nbq > (size_t)4 * T) return sg;  // pre-quantized entries per thread (PQ)
    sg.ok = true;
    sg.ng = ng;
    sg.kq = (uint32_t)kq;
    sg.nbq = (uint32_t)nbq;
    return sg;
}
TileGeo tile_geometry(const WDev &w, size_t m) {
    TileGeo none = {false, 0, 0, 0, 0};
    if (m < 1 || m > 8 || w.block > QPASS || w.block < 16) return none;
    const size_t tiles16 = w.n_pad / 16;
    // up to ~3 workgroups per CU (measured on MI355X; the rows of a multi-row
    // call are quantized once, before the launch)
    const size_t most = 768;
    uint32_t want = 0;
    while (want < 2 && (tiles16 >> want) > most) want++;
    for (int cs = (int)want; cs >= 0; cs--) {
        const TileGeo g = tile_geometry_cg(w, m, (uint32_t)cs);
        if (g.ok) return g;
    }
    return none;
}

RowShape row_shape(const WDev &w, size_t m, const TileGeo &sg, const EpArgs &ep) {
    RowShape r = {0, 0};
    const uint32_t grp = w.kind == W_Q2 ? Q2_GROUP : Q1_GROUP;
    if (!sg.ok || m < 1 || m > 8 || w.block != 128 || sg.ng > 4 ||
        w.n_pad != (((w.n ? w.n : 1u) + 127u) & ~(size_t)127u) || w.nchunks != (w.k + grp - 1) / grp)
        return r;
    const EpPick pk = pick_ep(ep);
    if (pk.v < 1 || pk.v > 3 || pk.act > 0xFF) return r;
    const uint32_t tiles = (uint32_t)(w.n_pad >> (4 + sg.cg_shift));
    const uint32_t grid = std::min<uint32_t>(tiles, (uint32_t)device_cus());
    const int tpw = grid ? (int)((tiles + grid - 1) / grid) : 0;
    const int mr = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    // one folding thread per (tile, row, column) of a workgroup
    if (tpw < 1 || tpw > 4 || (size_t)tpw * mr * (16u << sg.cg_shift) > (size_t)T ||
        row_lds_bytes(sg.kq, sg.nbq, 1u << sg.cg_shift, tpw, mr) > 150 * 1024)
        return r;
    r.grid = grid;
    r.tpw = tpw;
    return r;
}

// Bytes of the pre-quantized rows (q [m][kq], then s and sum(q) [m][nbq]).
size_t prequant_bytes(size_t m, size_t kq, size_t nbq) { return (m * kq + 255) / 256 * 256 + m * nbq * 8; }

}  // namespace

size_t lowbit_scratch_bytes(const WDev &w, size_t m, const EpArgs *ep) {
    const TileGeo sg = tile_geometry(w, m);
    if (sg.ok && ep && row_shape(w, m, sg, *ep).tpw > 0) return 0;  // lowbit_row quantizes in-kernel
    if (sg.ok) return m > 1 ? prequant_bytes(m, sg.kq, sg.nbq) : 0;
    const Geo ge = geometry(w, m);
    return (m * ge.kq + 255) / 256 * 256 + m * ge.nbq * 8;
}

hipError_t launch_lowbit_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                              const EpArgs &ep, void *scratch, hipStream_t s) {
    const TileGeo sg = tile_geometry(w, m);
    if (sg.ok) {
        const size_t cb = cell_grid_rows(w.nchunks) * w.n_pad * 64;
        if (m * w.k * 2 >= ((size_t)1 << 31) || cell_grid_rows(w.sc_rows) * w.n_pad * 2 >= ((size_t)1 << 31) ||
            cb >= ((size_t)1 << 31))
            return hipErrorInvalidValue;  // one buffer resource spans < 2 GiB
        LtArgs f = {};
        f.codes = w.codes;
        f.sc = w.scales;
        f.lhs = lhs;
        f.dst = dst;
        f.n = (uint32_t)w.n;
        f.k = (uint32_t)w.k;
        f.n_pad = (uint32_t)w.n_pad;
        f.m = (uint32_t)m;
        f.block_shift = ilog2(w.block);
        f.codebook = w.codebook;
        f.sc_rows = (uint32_t)w.sc_rows;
        f.ngroups = (uint32_t)w.nchunks;
        f.kq = sg.kq;
        f.nbq = sg.nbq;
        f.codes_bytes = (uint32_t)cb;
        f.cg_shift = sg.cg_shift;
        const int mr = m <= 2 ? (int)m : m <= 4 ? 4 : 8;
        const RowShape rs = row_shape(w, m, sg, ep);
        if (rs.tpw > 0)
            return w.kind == W_Q2 ? launch_row<2>(f, ep, sg.ng, rs, s) : launch_row<1>(f, ep, sg.ng, rs, s);
        if (m > 1) {
            f.q = (const int8_t *)scratch;
            f.qs = (const float *)((uint8_t *)scratch + (m * sg.kq + 255) / 256 * 256);
            f.qsum = (const int32_t *)(f.qs + m * sg.nbq);
            const dim3 grid((sg.kq + QPASS - 1) / QPASS, (uint32_t)m);
            if (w.kind == W_Q2)
                hipLaunchKernelGGL(lowbit_prequant<2>, grid, dim3(T), 0, s, lhs, f.m, f.k, f.kq, f.nbq,
                                   f.block_shift, (int8_t *)f.q, (float *)f.qs, (int32_t *)f.qsum);
            else
                hipLaunchKernelGGL(lowbit_prequant<1>, grid, dim3(T), 0, s, lhs, f.m, f.k, f.kq, f.nbq,
                                   f.block_shift, (int8_t *)f.q, (float *)f.qs, (int32_t *)f.qsum);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        if (w.kind == W_Q2) return launch_tile<2>(f, ep, mr, sg.ng, s);
        return launch_tile<1>(f, ep, mr, sg.ng, s);
    }
    const Geo ge = geometry(w, m);
    if (m * ge.kq >= ((size_t)1 << 31) || cell_grid_rows(w.sc_rows) * w.n_pad * 2 >= ((size_t)1 << 31))
        return hipErrorInvalidValue;  // one buffer resource spans < 2 GiB
    LbArgs g = {};
    g.codes = w.codes;
    g.sc = w.scales;
    g.dst = dst;
    g.n = (uint32_t)w.n;
    g.k = (uint32_t)w.k;
    g.n_pad = (uint32_t)w.n_pad;
    g.m = (uint32_t)m;
    g.block_shift = ilog2(w.block);
    g.codebook = w.codebook;
    g.kq = (uint32_t)ge.kq;
    g.nbq = (uint32_t)ge.nbq;
    g.sc_rows = (uint32_t)w.sc_rows;
    g.ngroups = (uint32_t)w.nchunks;
    g.seg_depths = (uint32_t)ge.seg;
    int8_t *q = (int8_t *)scratch;
    float *sp = (float *)((uint8_t *)scratch + (m * ge.kq + 255) / 256 * 256);
    int32_t *ap = (int32_t *)(sp + m * ge.nbq);
    g.q = q;
    g.s = sp;
    g.asum = ap;
    hipLaunchKernelGGL(lowbit_quant, dim3(g.nbq, (uint32_t)m), dim3(256), 0, s, lhs, g.k,
                       (uint32_t)w.block, g.nbq, q, sp, ap, g.kq);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int mr = rows_per_group(m);
    if (w.kind == W_Q2) return launch_kind<2>(g, ep, mr, s);
    return launch_kind<1>(g, ep, mr, s);
}

}  // namespace smg
