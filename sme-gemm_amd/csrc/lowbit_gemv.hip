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
    const rsrc_t sr = make_rsrc(g.sc, g.sc_rows * g.n_pad * 2u);
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
                                          lb_dword_offset<KIND>((size_t)sl * LB_SLAB + 16 * gq4, col, g.n_pad));
        }
        // scales of the 16 columns (32 bytes a block), activation scales, sums
        constexpr int RS = 4;  // up to 4 x 512 x 16 B = 32 KB of scale rows
        uint4 sreg[RS];
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const uint32_t i = t + T * r, bb = i / 2, half = i % 2;
            sreg[r] = bload16(sr, bb < nb ? ((b0 + bb) * g.n_pad + col0) * 2u + half * 16u : OOB);
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

}  // namespace

size_t lowbit_scratch_bytes(const WDev &w, size_t m) {
    const Geo ge = geometry(w, m);
    return (m * ge.kq + 255) / 256 * 256 + m * ge.nbq * 8;
}

hipError_t launch_lowbit_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                              const EpArgs &ep, void *scratch, hipStream_t s) {
    const Geo ge = geometry(w, m);
    if (m * ge.kq >= ((size_t)1 << 31) || w.sc_rows * w.n_pad * 2 >= ((size_t)1 << 31))
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
