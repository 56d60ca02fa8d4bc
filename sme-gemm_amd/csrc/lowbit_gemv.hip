// 2-bit / 1-bit int8 GEMV: matmul_q2 / matmul_q1 (+ _ep).
//
// Replaces csrc/gemm_q2.cc:48-429 (q2_quant, run_q2_gemv, Q2_FOLD) and is bit
// for bit the reference's portable result (src/kernels/lowbit/matmul.rs:354-398):
//   1. each row of A is quantized per K-block: amax = max|a| (NaN if any a is),
//      inv = amax > 0 ? 127/amax : 0, s = amax/127 (IEEE divides),
//      q = round_ties_even(a*inv) saturated to int8 (NaN -> 0);
//   2. exact i32 block sums sum_d q_d * value(d, j), value = codebook[code]
//      (Q2) or +-1 (Q1);
//   3. per column, in block order: total = fmaf(f32(sum), f32(scale)*s, total)
//      with the product scale*s rounded separately;
//   4. f16 RNE, then the op-graph.
// Integer sums are order-free, so the K split across lanes is exact; only the
// fold is sequential, done by one lane per (row, column) in block order.
//
// A workgroup owns 16 columns; 16 lanes per column split each pass along K.
// Q2 codes expand to int8 with one v_perm_b32 per 4 depths (codebook bytes as
// the table); Q1 signs expand to 0/1 bytes and use sum(q*(2b-1)) =
// 2*sum(q*b) - sum(q). Dot products are v_dot4_i32_i8.
#include "kernels.h"

namespace smg {

namespace {

constexpr int TN = 16;
constexpr int KL = 16;
constexpr int CPT = 8;  // max chunks per lane per pass
constexpr size_t AQ_BYTES = 32768;  // LDS for the pass's int8 activations
constexpr size_t S_BYTES = 32768;   // LDS for block sums

struct LbArgs {
    const uint8_t *codes;
    const uint16_t *sc;
    const uint16_t *lhs;
    uint16_t *dst;
    // pre-quantized activations (only when PREQ)
    const int8_t *gq;
    const float *gs;
    const int32_t *gasum;
    uint32_t n, k, n_pad, nchunks, m;
    uint32_t block_shift;
    uint32_t pd_shift;  // log2(depths per pass)
    uint32_t codebook;
    uint32_t nbk;
    uint32_t kq;        // row stride of gq
    uint32_t off_s, off_sa, off_asum;  // LDS layout (bytes)
};

template <int KIND>
struct Geo {
    static constexpr int CH = KIND == 2 ? 64 : 128;  // depths per 16-byte chunk
};

// Quantize rows [row0, row0+mr) over pass depths [p0, p1) into LDS.
// Every block of the pass lies inside it (pass length is a multiple of block).
__device__ void quantize_pass(const LbArgs &g, int mr, uint32_t row0, uint32_t p0, uint32_t p1,
                              int8_t *aq, float *sa, int32_t *asum, uint32_t pd) {
    const uint32_t block = 1u << g.block_shift;
    // lanes per (row, block) pair: each lane owns EL contiguous depths
    const uint32_t G = block / 16 < 64 ? (block / 16 > 0 ? block / 16 : 1) : 64;
    const uint32_t EL = block / G;  // 16 when block <= 1024
    const uint32_t nb = (p1 - p0 + block - 1) >> g.block_shift;
    const uint32_t npairs = (uint32_t)mr * nb;
    const uint32_t groups = 256 / G;
    const uint32_t t = threadIdx.x;
    const uint32_t gi = t / G, li = t % G;
    const rsrc_t ar = make_rsrc(g.lhs, g.m * g.k * 2u);
    const bool vec = (g.k & 7) == 0;
    for (uint32_t pr = gi; pr < ((npairs + groups - 1) / groups) * groups; pr += groups) {
        const bool live = pr < npairs;
        const uint32_t r = live ? pr / nb : 0, b = live ? pr % nb : 0;
        const uint32_t dstart = p0 + b * block + li * EL;
        // buffer loads: a dead pair (rows = 0) and depths past k read zero
        const uint32_t row = row0 + r, rows = live ? g.m : 0u;
        // amax with NaN propagation (matmul.rs:356-363)
        float amax = 0.0f;
        bool nan = false;
        for (uint32_t e0 = 0; e0 < EL; e0 += 8) {
            const uint4 v = load_row8(ar, row, rows, g.k, dstart + e0, vec);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = fabsf(f16_to_f32((uint16_t)(w4[e / 2] >> (16 * (e % 2)))));
                nan = nan || (x != x);
                amax = fmaxf(amax, x);
            }
        }
        for (uint32_t off = G / 2; off > 0; off >>= 1) {
            amax = fmaxf(amax, __shfl_xor(amax, off, G));
            nan = nan | (__shfl_xor((int)nan, off, G) != 0);
        }
        if (nan) amax = __builtin_nanf("");
        const float inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        const float s = __fdiv_rn(amax, 127.0f);
        int32_t qs = 0;
        for (uint32_t e0 = 0; e0 < EL; e0 += 8) {
            const uint4 v = load_row8(ar, row, rows, g.k, dstart + e0, vec);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
            uint32_t packed[2] = {0, 0};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = f16_to_f32((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
                const float qv = rintf(x * inv);
                const int qi = (qv != qv) ? 0 : (int)fminf(fmaxf(qv, -128.0f), 127.0f);
                qs += qi;
                packed[e / 4] |= ((uint32_t)(qi & 0xff)) << (8 * (e % 4));
            }
            if (live)
                *(uint2 *)(aq + (size_t)r * pd + (dstart - p0) + e0) = make_uint2(packed[0], packed[1]);
        }
        for (uint32_t off = G / 2; off > 0; off >>= 1) qs += __shfl_xor(qs, off, G);
        if (live && li == 0) {
            sa[r * (pd >> g.block_shift) + b] = s;
            asum[r * (pd >> g.block_shift) + b] = qs;
        }
    }
}

template <int KIND, int MR, bool PREQ>
__global__ void __launch_bounds__(256) lowbit_gemv_kernel(LbArgs g, EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int CH = Geo<KIND>::CH;
    const uint32_t pd = 1u << g.pd_shift;
    const uint32_t block = 1u << g.block_shift;
    // blocks per pass (>= 1; PREQ passes sit inside one block)
    const uint32_t nbp = pd >= block ? (pd >> g.block_shift) : 1;
    int8_t *aq = (int8_t *)smem;                  // [MR][pd]
    int32_t *S = (int32_t *)(smem + g.off_s);      // [nbp][MR][TN]
    float *sa = (float *)(smem + g.off_sa);        // [MR][nbp]
    int32_t *asum = (int32_t *)(smem + g.off_asum);  // [MR][nbp]

    const int t = threadIdx.x;
    const int c = t % TN;
    const int kl = t / TN;
    const uint32_t j = blockIdx.x * TN + c;
    const uint32_t row0 = blockIdx.y * MR;
    const int mr = (int)min((uint32_t)MR, g.m - row0);

    // fold lanes: one per (row, column)
    const bool folder = t < MR * TN;
    const int fr = t / TN;
    float total = 0.0f;

    const uint32_t chunks_per_pass = pd / CH;
    const uint32_t cpt = (chunks_per_pass + KL - 1) / KL;
    const uint32_t npass = (g.k + pd - 1) >> g.pd_shift;
    for (uint32_t pass = 0; pass < npass; pass++) {
        const uint32_t p0 = pass << g.pd_shift;
        const uint32_t p1 = min(p0 + pd, g.k);
        const uint32_t kc0 = p0 / CH;
        // 1. this lane's weight chunks, all loads issued up front
        uint4 wq[CPT];
#pragma unroll
        for (int q = 0; q < CPT; q++) {
            // branch-free: a chunk this lane does not own loads a valid
            // chunk (the last), and is never used
            const uint32_t kcl = kl * cpt + q;
            const uint32_t kc = kc0 + kcl;
            const bool own = q < (int)cpt && kcl < chunks_per_pass && kc < g.nchunks;
            const uint32_t kcc = own ? kc : g.nchunks - 1;
            wq[q] = *(const uint4 *)(g.codes + ((size_t)kcc * g.n_pad + j) * 16);
        }
        // 2. activations for the pass; zero the block sums
        __syncthreads();
        const bool block_starts = PREQ ? ((p0 & (block - 1)) == 0) : true;
        if (block_starts)
            for (uint32_t i = t; i < nbp * MR * TN; i += 256) S[i] = 0;
        if (!PREQ) {
            quantize_pass(g, mr, row0, p0, p1, aq, sa, asum, pd);
        } else {
            // copy the pass of the pre-quantized rows; block scale / sums
            for (uint32_t i = t * 4; i < (uint32_t)MR * pd; i += 256 * 4) {
                uint32_t r = i / pd, x = i % pd;
                uint32_t v = 0;
                if ((int)r < mr && p0 + x < g.k)
                    v = *(const uint32_t *)(g.gq + (size_t)(row0 + r) * g.kq + p0 + x);
                *(uint32_t *)(aq + r * pd + x) = v;
            }
            if (t < MR) {
                uint32_t blk = p0 >> g.block_shift;
                sa[t] = (t < mr) ? g.gs[(size_t)(row0 + t) * g.nbk + blk] : 0.0f;
                asum[t] = (t < mr) ? g.gasum[(size_t)(row0 + t) * g.nbk + blk] : 0;
            }
        }
        __syncthreads();
        // 3. exact block sums
        {
            int32_t part[MR];
#pragma unroll
            for (int r = 0; r < MR; r++) part[r] = 0;
            int cur = -1;  // block slot the partials belong to
#pragma unroll
            for (int q = 0; q < CPT; q++) {
                const uint32_t kcl = kl * cpt + q;
                if (q >= (int)cpt || kcl >= chunks_per_pass || kc0 + kcl >= g.nchunks) break;
                const uint32_t words[4] = {wq[q].x, wq[q].y, wq[q].z, wq[q].w};
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    constexpr int STEPS = KIND == 2 ? 4 : 8;   // 4-depth steps per dword
#pragma unroll
                    for (int i = 0; i < STEPS; i++) {
                        const uint32_t dl = kcl * CH + w * (4 * STEPS) + 4 * i;  // depth in pass
                        const int slot = PREQ ? 0 : (int)(dl >> g.block_shift);
                        if (slot != cur) {
                            if (cur >= 0) {
#pragma unroll
                                for (int r = 0; r < MR; r++)
                                    if (r < mr) atomicAdd(&S[(cur * MR + r) * TN + c], part[r]);
                            }
#pragma unroll
                            for (int r = 0; r < MR; r++) part[r] = 0;
                            cur = slot;
                        }
                        uint32_t wv;
                        if (KIND == 2) {
                            uint32_t sel = (words[w] >> (2 * i)) & 0x03030303u;
                            wv = __builtin_amdgcn_perm(g.codebook, g.codebook, sel);
                        } else {
                            wv = (words[w] >> i) & 0x01010101u;
                        }
#pragma unroll
                        for (int r = 0; r < MR; r++) {
                            const int32_t a4 = *(const int32_t *)(aq + r * pd + dl);
                            part[r] = __builtin_amdgcn_sdot4(a4, (int)wv, part[r], false);
                        }
                    }
                }
            }
            if (cur >= 0) {
#pragma unroll
                for (int r = 0; r < MR; r++)
                    if (r < mr) atomicAdd(&S[(cur * MR + r) * TN + c], part[r]);
            }
        }
        __syncthreads();
        // 4. fold the blocks that end in this pass, in block order
        const bool block_ends = PREQ ? (((p0 + pd) & (block - 1)) == 0 || p1 == g.k) : true;
        if (folder && fr < mr && block_ends) {
            const uint32_t nb_here = PREQ ? 1 : ((p1 - p0 + block - 1) >> g.block_shift);
            const uint32_t blk0 = p0 >> g.block_shift;
            for (uint32_t b = 0; b < nb_here; b++) {
                int32_t sum = S[(b * MR + fr) * TN + c];
                if (KIND == 1) sum = 2 * sum - asum[fr * nbp + b];
                const float f = (float)sum;
                const float wsc = f16_to_f32(g.sc[(size_t)(blk0 + b) * g.n_pad + j]);
                const float sc = wsc * sa[fr * nbp + b];
                total = fmaf(f, sc, total);
            }
        }
    }
    if (folder && fr < mr && j < g.n) {
        const uint32_t row = row0 + fr;
        g.dst[(size_t)row * g.n + j] = finish<false>(ep, total, row, j, g.n);
    }
}

// Stand-alone quantization for blocks too long to quantize inside one pass:
// one workgroup per (row, block). Writes q (int8, row stride kq), s, asum.
__global__ void __launch_bounds__(256) lowbit_quant_kernel(const uint16_t *lhs, uint32_t k,
                                                           uint32_t block, uint32_t nbk,
                                                           int8_t *q, float *s, int32_t *asum,
                                                           uint32_t kq) {
    __shared__ float red[256];
    __shared__ int redn[256];
    const uint32_t b = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    const uint32_t d0 = b * block, d1 = min(d0 + block, k);
    const uint16_t *src = lhs + (size_t)r * k;
    float amax = 0.0f;
    int nan = 0;
    for (uint32_t d = d0 + t; d < d1; d += 256) {
        float x = fabsf(f16_to_f32(src[d]));
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
    for (uint32_t d = d0 + t; d < d0 + block; d += 256) {
        int qi = 0;
        if (d < d1) {
            float v = rintf(f16_to_f32(src[d]) * inv);
            qi = (v != v) ? 0 : (int)fminf(fmaxf(v, -128.0f), 127.0f);
        }
        if (d < kq) q[(size_t)r * kq + d] = (int8_t)qi;
        qs += qi;
    }
    redn[t] = qs;
    __syncthreads();
    for (uint32_t off = 128; off > 0; off >>= 1) {
        if (t < off) redn[t] += redn[t + off];
        __syncthreads();
    }
    if (t == 0) {
        s[(size_t)r * nbk + b] = __fdiv_rn(amax, 127.0f);
        asum[(size_t)r * nbk + b] = redn[0];
    }
}

inline uint32_t ilog2(size_t x) { return (uint32_t)(63 - __builtin_clzll(x)); }

// Depths per pass: a power of two holding whole blocks when it can, within
// the LDS budgets for int8 activations (AQ_BYTES) and block sums (S_BYTES),
// and at most CPT chunks per lane.
inline size_t pass_depths(int kind, size_t block, int mr, size_t k) {
    const size_t ch = kind == 2 ? 64 : 128;
    size_t pd = (size_t)KL * CPT * ch;
    // no longer than K needs (fewer idle chunk slots per lane)
    while (pd / 2 >= k && pd / 2 >= ch && pd / 2 >= block) pd >>= 1;
    while (pd * mr > AQ_BYTES) pd >>= 1;
    while (pd >= block && (pd / block) * mr * TN * 4 > S_BYTES) pd >>= 1;
    if (pd / block > 512) pd = 512 * block;
    if (pd < ch) pd = ch;
    return pd;
}

template <int KIND, int MR>
hipError_t launch_kind(LbArgs g, const EpArgs &ep, bool preq, hipStream_t s) {
    const size_t pd = (size_t)1 << g.pd_shift, block = (size_t)1 << g.block_shift;
    const size_t nbp = pd >= block ? pd / block : 1;
    g.off_s = (uint32_t)(((size_t)MR * pd + 15) / 16 * 16);
    g.off_sa = g.off_s + (uint32_t)(nbp * MR * TN * 4);
    g.off_asum = g.off_sa + (uint32_t)(MR * nbp * 4);
    const size_t lds = g.off_asum + MR * nbp * 4;
    dim3 grid(g.n_pad / TN, (g.m + MR - 1) / MR);
    if (preq)
        hipLaunchKernelGGL((lowbit_gemv_kernel<KIND, MR, true>), grid, dim3(256), lds, s, g, ep);
    else
        hipLaunchKernelGGL((lowbit_gemv_kernel<KIND, MR, false>), grid, dim3(256), lds, s, g, ep);
    return hipGetLastError();
}

template <int KIND>
hipError_t launch_rows(LbArgs g, const EpArgs &ep, bool preq, int mr, hipStream_t s) {
    if (mr <= 1) return launch_kind<KIND, 1>(g, ep, preq, s);
    if (mr <= 2) return launch_kind<KIND, 2>(g, ep, preq, s);
    if (mr <= 4) return launch_kind<KIND, 4>(g, ep, preq, s);
    return launch_kind<KIND, 8>(g, ep, preq, s);
}

inline int rows_per_group(size_t m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; }

}  // namespace

size_t lowbit_scratch_bytes(const WDev &w, size_t m) {
    const int mr = rows_per_group(m);
    const size_t pd = pass_depths(w.kind, w.block, mr, w.k);
    if (pd >= w.block) return 0;
    const size_t nbk = (w.k + w.block - 1) / w.block;
    const size_t kq = nbk * w.block;
    return ((m * kq + 255) / 256) * 256 + m * nbk * 8;
}

hipError_t launch_lowbit_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                              const EpArgs &ep, void *scratch, hipStream_t s) {
    const int mr = rows_per_group(m);
    const size_t pd = pass_depths(w.kind, w.block, mr, w.k);
    const bool preq = pd < w.block;
    LbArgs g = {};
    g.codes = w.codes;
    g.sc = w.scales;
    g.lhs = lhs;
    g.dst = dst;
    g.n = (uint32_t)w.n;
    g.k = (uint32_t)w.k;
    g.n_pad = (uint32_t)w.n_pad;
    g.nchunks = (uint32_t)w.nchunks;
    g.m = (uint32_t)m;
    g.block_shift = ilog2(w.block);
    g.pd_shift = ilog2(pd);
    g.codebook = w.codebook;
    g.nbk = (uint32_t)((w.k + w.block - 1) / w.block);
    if (preq) {
        const size_t kq = (size_t)g.nbk * w.block;
        g.kq = (uint32_t)kq;
        int8_t *q = (int8_t *)scratch;
        float *sp = (float *)((uint8_t *)scratch + ((m * kq + 255) / 256) * 256);
        int32_t *ap = (int32_t *)(sp + m * g.nbk);
        g.gq = q;
        g.gs = sp;
        g.gasum = ap;
        hipLaunchKernelGGL(lowbit_quant_kernel, dim3(g.nbk, (uint32_t)m), dim3(256), 0, s, lhs,
                           g.k, (uint32_t)w.block, g.nbk, q, sp, ap, g.kq);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (w.kind == W_Q2) return launch_rows<2>(g, ep, preq, mr, s);
    return launch_rows<1>(g, ep, preq, mr, s);
}

}  // namespace smg
