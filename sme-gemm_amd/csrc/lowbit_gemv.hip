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
// Layout of the work: one wave owns 16 output columns over all of K, so each
// output's fold is a sequential chain inside one lane. The block sums come
// from v_mfma_i32_16x16x64_i8 (exact i32): A operand = 16 columns x 64 depths
// of weights expanded to int8 (Q2: one v_perm_b32 per 4 depths with the
// codebook bytes as the table; Q1: sign bits to 0/1 bytes, using
// sum(q*(2b-1)) = 2*sum(q*b) - sum(q)), B operand = 64 depths x up to 16
// quantized activation rows from LDS. A workgroup of W waves shares the
// quantized activations. K is processed in segments whose weight loads are
// all issued before the segment's activations are quantized.
#include "kernels.h"

namespace smg {

namespace {

constexpr int NGMAX = 16;            // 16-byte weight groups per lane per segment
constexpr int AQ_BUDGET = 32768;     // LDS bytes of int8 activations per segment

__host__ __device__ constexpr int group_depths(int kind) { return kind == 2 ? Q2_GROUP : Q1_GROUP; }
__host__ __device__ constexpr int seg_depths(int kind, int mr) {
    return NGMAX * group_depths(kind) < AQ_BUDGET / mr ? NGMAX * group_depths(kind)
                                                       : AQ_BUDGET / mr;
}

struct LbArgs {
    const uint8_t *codes;
    const uint16_t *sc;
    const uint16_t *lhs;
    uint16_t *dst;
    // pre-quantized activations (only for blocks longer than a segment)
    const int8_t *gq;
    const float *gs;
    const int32_t *gasum;
    uint32_t n, k, n_pad, ngroups, m;
    uint32_t block_shift;
    uint32_t codebook;
    uint32_t nbk;
    uint32_t kq;  // row stride of gq
    uint32_t off_scl, off_sa, off_asum, nbs;  // LDS layout; block slots per segment
    uint32_t sc_rows;
};

__device__ __forceinline__ uint16_t half_of(const uint4 &v, int e) {
    const uint32_t w = e / 2 == 0 ? v.x : e / 2 == 1 ? v.y : e / 2 == 2 ? v.z : v.w;
    return (uint16_t)(w >> (16 * (e % 2)));
}

template <int KIND, int W, int MR, bool PREQ>
__global__ void __launch_bounds__(W * 64) lowbit_mfma(LbArgs g, EpArgs ep) {
    constexpr int T = W * 64;
    constexpr int GRP = group_depths(KIND);
    constexpr int SEG = seg_depths(KIND, MR);
    constexpr int SPG = GRP / LB_SLAB;  // slabs per 16-byte group (4 or 8)
    constexpr int E = (MR * SEG) / T;   // activations each thread quantizes
    constexpr int NCH = E / 16;         // 16-element chunks per thread (blocks are >= 16)
    static_assert(E >= 16 && E % 16 == 0, "segment too short for the workgroup");

    extern __shared__ __align__(16) uint8_t smem[];
    int8_t *aq = (int8_t *)smem;                     // [MR][SEG]
    uint16_t *scl = (uint16_t *)(smem + g.off_scl);   // [nbs][16W]
    float *sa = (float *)(smem + g.off_sa);           // [MR][nbs]
    int32_t *asum = (int32_t *)(smem + g.off_asum);   // [MR][nbs]

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int gq4 = lane >> 4, c = lane & 15;  // quarter; column (A) / row (B)
    const uint32_t colw = blockIdx.x * 16 * W;  // first column of the workgroup
    const uint32_t col = colw + wave * 16 + c;  // this lane's weight column (< n_pad)
    const uint32_t row0 = blockIdx.y * MR;
    const uint32_t mr = min((uint32_t)MR, g.m - row0);
    const uint32_t block = 1u << g.block_shift;

    float total[4] = {0.f, 0.f, 0.f, 0.f};
    int4_t acc = {0, 0, 0, 0};

    const rsrc_t ar = make_rsrc(g.lhs, g.m * g.k * 2u);
    const bool vec = (g.k & 7) == 0;
    const uint32_t nseg = (g.k + SEG - 1) / SEG;
    for (uint32_t seg = 0; seg < nseg; seg++) {
        const uint32_t d0 = seg * SEG;
        const uint32_t dl = min((uint32_t)SEG, g.k - d0);
        // -- 0. this thread's activation run first (vmcnt retires in issue order)
        const uint32_t er = (t * E) / SEG, ex = (t * E) % SEG;  // row, depth in segment
        uint4 areg[PREQ ? 1 : E / 8];
        if (!PREQ) {
#pragma unroll
            for (int q = 0; q < E / 8; q++)
                areg[q] = load_row8(ar, row0 + er, row0 + mr, g.k, d0 + ex + 8 * q, vec);
        }
        // -- 0b. block scales of the workgroup's columns for the segment's
        //        blocks: rows b0.., 32W contiguous bytes each, 16 bytes a load
        const uint32_t b0 = d0 >> g.block_shift;  // first block of the segment
        const uint32_t nbs_here = PREQ ? 1 : (dl + block - 1) >> g.block_shift;
        constexpr int SCL_LOADS = (SEG / 16) * 2 * W / T > 0 ? (SEG / 16) * 2 * W / T : 1;
        const rsrc_t sr = make_rsrc(g.sc, g.sc_rows * g.n_pad * 2u);
        uint4 sreg[SCL_LOADS];
#pragma unroll
        for (int r = 0; r < SCL_LOADS; r++) {
            const uint32_t i = t + T * r, lb = i / (2 * W), part = i % (2 * W);
            sreg[r] = bload16(sr, lb < nbs_here ? ((b0 + lb) * g.n_pad + colw) * 2u + part * 16u : OOB);
        }
        // -- 1. the segment's weights: group q0 + u, quarter gq4, column col
        //       (a group past the segment reloads the last one: no branch)
        const uint32_t q0 = d0 / GRP;
        const uint32_t ng = (dl + GRP - 1) / GRP;
        uint4 wq[NGMAX];
#pragma unroll
        for (int u = 0; u < NGMAX; u++) {
            const uint32_t qq = (uint32_t)u < ng ? q0 + u : q0 + ng - 1;
            wq[u] = *(const uint4 *)(g.codes + (((size_t)qq * g.n_pad + col) * 4 + gq4) * 16);
        }
        __syncthreads();  // the previous segment is done with LDS
        if (!PREQ) {
            // -- 2. quantize. A block covers S = L/16 consecutive chunks of one
            //       thread (L = min(E, block)), spread over G = block/L threads.
            const uint32_t L = (uint32_t)E < block ? (uint32_t)E : block;
            const uint32_t S = L / 16, G = block / L;
            float cm[NCH];
            bool cn[NCH];
#pragma unroll
            for (int h = 0; h < NCH; h++) {
                float mx = 0.0f;
                bool nn = false;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float x = fabsf(f16_to_f32(half_of(areg[2 * h + e / 8], e % 8)));
                    nn = nn || (x != x);
                    mx = fmaxf(mx, x);
                }
                cm[h] = mx;
                cn[h] = nn;
            }
            // combine the chunks of a block (butterfly over aligned groups of S)
#pragma unroll
            for (int off = 1; off < NCH; off <<= 1) {
                if ((uint32_t)off < S) {
                    float nm[NCH];
                    bool nnn[NCH];
#pragma unroll
                    for (int h = 0; h < NCH; h++) {
                        nm[h] = fmaxf(cm[h], cm[h ^ off]);
                        nnn[h] = cn[h] || cn[h ^ off];
                    }
#pragma unroll
                    for (int h = 0; h < NCH; h++) {
                        cm[h] = nm[h];
                        cn[h] = nnn[h];
                    }
                }
            }
            // and across the G threads of a long block (then S covers all chunks)
            for (uint32_t off = G / 2; off > 0; off >>= 1) {
                const float o = __shfl_xor(cm[0], off, G);
                const int on = __shfl_xor((int)cn[0], off, G);
#pragma unroll
                for (int h = 0; h < NCH; h++) {
                    cm[h] = fmaxf(cm[h], o);
                    cn[h] = cn[h] || (on != 0);
                }
            }
            int32_t qs[NCH];
#pragma unroll
            for (int h = 0; h < NCH; h++) {
                const float amax = cn[h] ? __builtin_nanf("") : cm[h];
                cm[h] = amax;
                const float inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                uint32_t packed[4] = {0, 0, 0, 0};
                int32_t sum = 0;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float x = f16_to_f32(half_of(areg[2 * h + e / 8], e % 8));
                    const float qv = rintf(x * inv);
                    const int qi = (qv != qv) ? 0 : (int)fminf(fmaxf(qv, -128.0f), 127.0f);
                    sum += qi;
                    packed[e / 4] |= ((uint32_t)(qi & 0xff)) << (8 * (e % 4));
                }
                qs[h] = sum;
                *(uint4 *)(aq + er * SEG + ex + 16 * h) =
                    make_uint4(packed[0], packed[1], packed[2], packed[3]);
            }
#pragma unroll
            for (int off = 1; off < NCH; off <<= 1) {
                if ((uint32_t)off < S) {
                    int32_t ns[NCH];
#pragma unroll
                    for (int h = 0; h < NCH; h++) ns[h] = qs[h] + qs[h ^ off];
#pragma unroll
                    for (int h = 0; h < NCH; h++) qs[h] = ns[h];
                }
            }
            for (uint32_t off = G / 2; off > 0; off >>= 1) {
                const int o = __shfl_xor(qs[0], off, G);
#pragma unroll
                for (int h = 0; h < NCH; h++) qs[h] += o;
            }
            if ((t % G) == 0) {
#pragma unroll
                for (int h = 0; h < NCH; h++) {
                    if ((h % S) == 0) {
                        const uint32_t lb = (ex + 16 * h) >> g.block_shift;  // block in segment
                        sa[er * g.nbs + lb] = __fdiv_rn(cm[h], 127.0f);
                        asum[er * g.nbs + lb] = qs[h];
                    }
                }
            }
        } else {
            // blocks longer than a segment: q, s, sum(q) come from the
            // stand-alone quantizer; copy this segment's q
            const rsrc_t qr = make_rsrc(g.gq, g.m * g.kq);
            for (uint32_t i = t * 16; i < (uint32_t)MR * SEG; i += T * 16) {
                const uint32_t r = i / SEG, x = i % SEG;
                *(uint4 *)(aq + r * SEG + x) =
                    bload16(qr, (r < mr && d0 + x < g.k) ? (row0 + r) * g.kq + d0 + x : OOB);
            }
            if (t < MR) {
                sa[t] = (uint32_t)t < mr ? g.gs[(size_t)(row0 + t) * g.nbk + b0] : 0.0f;
                asum[t] = (uint32_t)t < mr ? g.gasum[(size_t)(row0 + t) * g.nbk + b0] : 0;
            }
        }
#pragma unroll
        for (int r = 0; r < SCL_LOADS; r++) {
            const uint32_t i = t + T * r, lb = i / (2 * W), part = i % (2 * W);
            if (lb < nbs_here) *(uint4 *)(scl + lb * 16 * W + part * 8) = sreg[r];
        }
        __syncthreads();
        // -- 3. block sums on the matrix cores, folded in block order
        const uint32_t nslab = (dl + LB_SLAB - 1) / LB_SLAB;
        const uint32_t parts = block < (uint32_t)LB_SLAB ? LB_SLAB / block : 1;
        const bool row_live = (uint32_t)c < mr;
#pragma unroll
        for (int u = 0; u < NGMAX; u++) {
            if ((uint32_t)u * SPG >= nslab) break;  // uniform
            const uint32_t words[4] = {wq[u].x, wq[u].y, wq[u].z, wq[u].w};
#pragma unroll
            for (int sl = 0; sl < SPG; sl++) {
                const uint32_t s = u * SPG + sl;  // slab within the segment
                if (s >= nslab) break;            // uniform
                // A operand: this lane's 16 depths (quarter gq4) of slab s as int8
                int4_t wa;
                if (KIND == 2) {
                    const uint32_t wd = words[sl];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        wa[i] = (int)__builtin_amdgcn_perm(g.codebook, g.codebook,
                                                           (wd >> (2 * i)) & 0x03030303u);
                } else {
                    const uint32_t wd = words[sl / 2];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        wa[i] = (int)((wd >> (4 * (sl % 2) + i)) & 0x01010101u);
                }
                // B operand: activation row c, the same 16 depths
                int4_t ab = {0, 0, 0, 0};
                if (row_live) ab = *(const int4_t *)(aq + c * SEG + s * LB_SLAB + 16 * gq4);
                for (uint32_t p = 0; p < parts; p++) {
                    // blocks shorter than a slab: one MFMA per block, the other
                    // quarters' activations masked to zero
                    int4_t abp = ab;
                    if (parts > 1 && (uint32_t)(16 * gq4) / block != p) abp = (int4_t){0, 0, 0, 0};
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa, abp, acc, 0, 0, 0);
                    bool ends;
                    uint32_t lb;
                    if (PREQ) {
                        ends = s + 1 == nslab && (((d0 + dl) & (block - 1)) == 0 || d0 + dl == g.k);
                        lb = 0;
                    } else if (parts > 1) {
                        ends = true;
                        lb = (s * LB_SLAB + p * block) >> g.block_shift;
                    } else {
                        ends = (((s + 1) * LB_SLAB) & (block - 1)) == 0 || s + 1 == nslab;
                        lb = (s * LB_SLAB) >> g.block_shift;
                    }
                    if (ends) {  // uniform
                        const float sav = sa[c * g.nbs + lb];
                        const int32_t as = asum[c * g.nbs + lb];
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const int32_t sum = KIND == 1 ? 2 * acc[v] - as : acc[v];
                            const float wsc = f16_to_f32(scl[lb * 16 * W + wave * 16 + 4 * gq4 + v]);
                            const float scv = wsc * sav;
                            total[v] = fmaf((float)sum, scv, total[v]);
                        }
                        acc = (int4_t){0, 0, 0, 0};
                    }
                }
            }
        }
    }
    // lane holds outputs (row c, columns 4*gq4 + v of its wave's 16)
    if ((uint32_t)c < mr) {
        const uint32_t row = row0 + c;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint32_t j = colw + wave * 16 + 4 * gq4 + v;
            if (j < g.n) g.dst[(size_t)row * g.n + j] = finish<false>(ep, total[v], row, j, g.n);
        }
    }
}

// Stand-alone quantization for blocks longer than a segment: one workgroup
// per (row, block). Writes q (int8, row stride kq), s and sum(q).
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
    for (uint32_t d = d0 + t; d < d0 + block; d += 256) {
        int qi = 0;
        if (d < d1) {
            const float v = rintf(f16_to_f32(src[d]) * inv);
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

inline int rows_per_group(size_t m) {
    return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16;
}
inline int waves_for(size_t m) { return m <= 2 ? 2 : 4; }

template <int KIND, int W, int MR>
hipError_t launch_t(LbArgs g, const EpArgs &ep, bool preq, hipStream_t s) {
    constexpr int SEG = seg_depths(KIND, MR);
    const size_t block = (size_t)1 << g.block_shift;
    const size_t nbs = (size_t)SEG >= block ? SEG / block : 1;
    g.nbs = (uint32_t)nbs;
    g.off_scl = (uint32_t)((size_t)MR * SEG);
    g.off_sa = g.off_scl + (uint32_t)((nbs * 16 * W * 2 + 15) / 16 * 16);
    g.off_asum = g.off_sa + (uint32_t)(MR * nbs * 4);
    const size_t lds = g.off_asum + MR * nbs * 4;
    static bool attr = false;  // benign race: every setter writes the same value
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)lowbit_mfma<KIND, W, MR, true>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)lowbit_mfma<KIND, W, MR, false>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const dim3 grid((unsigned)((g.n + 16 * W - 1) / (16 * W)), (unsigned)((g.m + MR - 1) / MR));
    if (preq)
        hipLaunchKernelGGL((lowbit_mfma<KIND, W, MR, true>), grid, dim3(W * 64), lds, s, g, ep);
    else
        hipLaunchKernelGGL((lowbit_mfma<KIND, W, MR, false>), grid, dim3(W * 64), lds, s, g, ep);
    return hipGetLastError();
}

template <int KIND, int W>
hipError_t launch_rows(LbArgs g, const EpArgs &ep, bool preq, int mr, hipStream_t s) {
    if (mr <= 1) return launch_t<KIND, W, 1>(g, ep, preq, s);
    if (mr <= 2) return launch_t<KIND, W, 2>(g, ep, preq, s);
    if (mr <= 4) return launch_t<KIND, W, 4>(g, ep, preq, s);
    if (mr <= 8) return launch_t<KIND, W, 8>(g, ep, preq, s);
    return launch_t<KIND, W, 16>(g, ep, preq, s);
}

template <int KIND>
hipError_t launch_kind(LbArgs g, const EpArgs &ep, bool preq, size_t m, hipStream_t s) {
    const int mr = rows_per_group(m);
    if (waves_for(m) == 2) return launch_rows<KIND, 2>(g, ep, preq, mr, s);
    return launch_rows<KIND, 4>(g, ep, preq, mr, s);
}

size_t seg_for(int kind, size_t m) { return (size_t)seg_depths(kind, rows_per_group(m)); }

}  // namespace

size_t lowbit_scratch_bytes(const WDev &w, size_t m) {
    if (seg_for(w.kind, m) >= w.block) return 0;
    const size_t nbk = (w.k + w.block - 1) / w.block;
    const size_t kq = nbk * w.block;
    return ((m * kq + 255) / 256) * 256 + m * nbk * 8;
}

hipError_t launch_lowbit_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                              const EpArgs &ep, void *scratch, hipStream_t s) {
    if (m * w.k * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;  // buffer range
    const bool preq = seg_for(w.kind, m) < w.block;
    LbArgs g = {};
    g.codes = w.codes;
    g.sc = w.scales;
    g.lhs = lhs;
    g.dst = dst;
    g.n = (uint32_t)w.n;
    g.k = (uint32_t)w.k;
    g.n_pad = (uint32_t)w.n_pad;
    g.ngroups = (uint32_t)w.nchunks;
    g.m = (uint32_t)m;
    g.block_shift = ilog2(w.block);
    g.codebook = w.codebook;
    g.nbk = (uint32_t)((w.k + w.block - 1) / w.block);
    g.sc_rows = (uint32_t)w.sc_rows;
    if (w.sc_rows * w.n_pad * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    if (preq) {
        const size_t kq = (size_t)g.nbk * w.block;
        if (m * kq >= ((size_t)1 << 31)) return hipErrorInvalidValue;
        g.kq = (uint32_t)kq;
        int8_t *q = (int8_t *)scratch;
        float *sp = (float *)((uint8_t *)scratch + ((m * kq + 255) / 256) * 256);
        int32_t *ap = (int32_t *)(sp + m * g.nbk);
        g.gq = q;
        g.gs = sp;
        g.gasum = ap;
        hipLaunchKernelGGL(lowbit_quant_kernel, dim3(g.nbk, (uint32_t)m), dim3(256), 0, s, lhs,
                           g.k, (uint32_t)w.block, g.nbk, q, sp, ap, g.kq);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (w.kind == W_Q2) return launch_kind<2>(g, ep, preq, m, s);
    return launch_kind<1>(g, ep, preq, m, s);
}

}  // namespace smg
