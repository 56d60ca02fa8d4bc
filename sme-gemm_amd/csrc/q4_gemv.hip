// Q4 GEMV for decode-shaped calls (m <= 8): C = ep(A @ dequant(B)).
//
// Replaces the SME GEMV of csrc/gemm_f16f16_q4.h:174-433 (run_q4_gemv1 /
// run_q4_gemv) and its bf16 twin csrc/gemm_b16b16_q4.h:171. Numerics follow
// the portable path the reference falls back to
// (src/kernels/q4/matmul.rs:91-102 -> src/reference.rs:349-387): every weight
// is rounded once to the output type (f16: RNE of scale*code [+ min]; bf16:
// through f32, weights.rs:198-201), products are exact in f32 and summed in
// f32 (split over K, so the sum order differs: tolerance-checked), the sum is
// rounded to f16/bf16 and the op-graph runs on that rounded value.
//
// The call is HBM-bound (0.5625 B of weights per MAC at block 32). Two kernels:
//
// q4_gemv_mfma (block >= 32, so one scale and min per chunk; f16 or bf16,
// scale-only or affine -- f16 scale-only is the decode configuration):
//   a workgroup of 8 waves owns 16 output columns; wave w takes every 8th
//   group of 4 chunks (128 depths). Lane (g = lane/16, c = lane%16) loads the
//   16-byte chunk g of column c, so a wave load reads one contiguous 1 KB run
//   of the blocked layout (common.cuh), and every lane issues all its weight loads
//   before it waits. Each
//   dword (8 depths) dequantizes to 8 f16 weights -- v_bfi_b32 puts the
//   nibble under an f16 exponent, a packed subtract leaves the exact code, a
//   packed multiply by the scale is the reference's single RNE rounding -- and
//   feeds one v_mfma_f32_16x16x32_f16 as the A operand (16 columns x 32
//   depths), with up to 16 activation rows as the B operand. The matrix core
//   does the dot products, so VALU work is the dequant alone. Affine weights
//   take one packed fma (scale*code + min, one rounding) in place of the
//   multiply; bf16 weights are formed in f32 (exact product, plus the min)
//   and rounded to bf16 in pairs, then feed v_mfma_f32_16x16x32_bf16. The 8
//   waves' partial 16x16 tiles are summed through LDS in a fixed order.
//
// q4_gemv_kernel (blocks shorter than a chunk, and K = 0): 16 columns x
//   16 lanes along K per workgroup, weights rounded per value, dot products on
//   VALU. All loads are branch-free (clamped address, then a select) so they
//   stay in flight together.
#include "q4_gemv_core.cuh"

namespace smg {

namespace {

// ---------------------------------------------------------------------------
// MFMA GEMV (fast path): the shared main loop (q4_gemv_core.cuh) over rows of
// f16 activations, then the 8 waves' partial tiles summed through LDS in a
// fixed order and the op-graph at the store.
// ---------------------------------------------------------------------------
// rows staged per segment (1, 2, 4, 8); chained call; bf16 activations and
// weights; Q4_1 (affine) weights
template <int MR, bool CHAIN, bool BF16 = false, bool AFFINE = false>
__global__ void __launch_bounds__(MF_WAVES * 64) q4_gemv_mfma(Q4GemvArgs g, EpArgs ep, ChainArgs ch) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *a_lds = (uint16_t *)smem;          // [MR][MF_SEG]
    float *red = (float *)smem;                   // reused: [MF_WAVES][16 cols][MR]

    const int t = threadIdx.x;
    const uint32_t tile = xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t col = tile * 16 + (t & 15);    // < n_pad
    bool timed_out = false;  // chained: a wait for A expired (uniform)
    constexpr int U = MR > 8 ? 2 : MF_U;  // 16 rows: half segments (64 KB staged)
    const SrcRows<MR, U * 1024> src(g.lhs, g.m, g.k);
    const float4_t acc = q4_mfma_mainloop<MR, CHAIN, SrcRows<MR, U * 1024>, true, BF16, AFFINE, U>(
        g, src, ch, a_lds, col, timed_out);
    q4_mfma_reduce<MR>(acc, red);
    if (t < 16 * MR) {
        const int cc = t / MR, r = t % MR;
        const float total = tile_total<MR>(red, cc, r);
        const uint32_t j = tile * 16 + cc;
        if (!timed_out && r < (int)g.m && j < g.n) g.dst[(size_t)r * g.n + j] = finish<BF16>(ep, total, r, j, g.n);
    }
    if constexpr (CHAIN) {
        if (timed_out && t == 0) __hip_atomic_store(ch.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (ch.done) {
            // one count per workgroup, a release that writes wave 0's stores
            // back (a wave's release waits for all of its own stores); a
            // second storing wave (8 rows) writes its own back first. The
            // last workgroup to count publishes.
            if (t >= 64 && t < 16 * MR) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __syncthreads();
            if (t == 0) {
                const uint32_t prev =
                    __hip_atomic_fetch_add(ch.sync, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                if (prev == gridDim.x - 1) {
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    const bool bad = __hip_atomic_load(ch.sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
                    __hip_atomic_store(ch.sync, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (!bad) __hip_atomic_store(ch.done, ch.done_value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMV, wave-staged (the unchained calls): the first 14 argument dwords
// -- everything the loads need -- are what the dispatcher preloads into SGPRs
// (this file is compiled with kernarg preloading), so a wave's first loads do
// not wait on a kernel-argument fetch; the op-graph arguments that follow are
// read only at the store, and only when the op-graph has nodes: misc = m |
// n_nodes << 8 carries its length in a preloaded dword, so a plain call's
// store reads no kernel argument (a scalar load of a line no earlier
// instruction touched would otherwise stand between every workgroup's
// reduction and its store). Each wave stages its own activations
// (q4_wave_loop), so the one workgroup barrier is the partial-tile
// reduction's. Block 32, k a multiple of 8 (16-byte activation rows), grids
// under 2 GiB.
// ---------------------------------------------------------------------------
template <int MR, bool BF16, bool AFFINE>
__global__ void __launch_bounds__(MF_WAVES * 64)
    q4_gemv_wave(const uint8_t *nib, const uint16_t *sc, const uint16_t *lhs, uint16_t *dst, uint32_t n_pad,
                 uint32_t nchunks, uint32_t k, uint32_t n, uint32_t tiles, uint32_t misc, const uint16_t *mn,
                 EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *wlds = (uint16_t *)smem + (threadIdx.x >> 6) * (MR * 512);  // [MR][4 runs][128]
    float *red = (float *)(smem + MF_WAVES * MR * 1024);                   // [MF_WAVES][16 cols][MR]
    const int t = threadIdx.x;
    const uint32_t tile = xcd_tile(blockIdx.x, tiles);
    const uint32_t col = tile * 16 + (t & 15);  // < n_pad
    const uint32_t m = misc & 0xFF, n_nodes = misc >> 8;
    const uint32_t grid_rows = (nchunks + 3) & ~3u;  // the nibble and (block 32) scale grids' rows
    Q4WaveArgs g;
    g.nr = make_rsrc(nib, grid_rows * n_pad * 16u);
    g.sr = make_rsrc(sc, grid_rows * n_pad * 2u);
    g.mr = make_rsrc(mn, AFFINE ? grid_rows * n_pad * 2u : 0u);
    g.ar = make_rsrc(lhs, m * k * 2u);
    g.n_pad = n_pad;
    g.nchunks = nchunks;
    g.k = k;
    g.m = m;
    const float4_t acc = q4_wave_loop<MR, BF16, AFFINE>(g, wlds, col);
    const int lane = t & 63, wave = t >> 6, c = lane & 15, grp = lane >> 4;
    if (c < MR) {
#pragma unroll
        for (int v = 0; v < 4; v++) red[(wave * 16 + 4 * grp + v) * MR + c] = acc[v];
    }
    __syncthreads();
    if (t < 16 * MR) {
        const int cc = t / MR, r = t % MR;
        const float total = tile_total<MR>(red, cc, r);
        const uint32_t j = tile * 16 + cc;
        if (r < (int)m && j < n)
            dst[(size_t)r * n + j] = n_nodes == 0 ? from_f32<BF16>(total) : finish<BF16>(ep, total, r, j, n);
    }
}

// ---------------------------------------------------------------------------
// Generic GEMV (blocks below 32: scales vary inside a chunk; K = 0)
// ---------------------------------------------------------------------------
constexpr int TN = 16;        // output columns per workgroup
constexpr int KL = 16;        // lanes along K per column
constexpr int P = 8;          // chunks per lane per pass
constexpr int PASS_CH = KL * P;            // chunks per pass
constexpr int PASS_D = PASS_CH * Q4_CHUNK; // depths per pass (4096)

// Two consecutive depths' weights as a packed pair of 16-bit values: the
// exact reference roundings, computed per value.
template <bool BF16, bool AFFINE>
__device__ __forceinline__ uint32_t deq_pair_generic(int c0, int c1, uint16_t s0, uint16_t s1,
                                                     uint16_t m0, uint16_t m1) {
    uint16_t w0, w1;
    if (!AFFINE) {
        // scale*code is exact in f32 (11-bit x 4-bit), so one rounding to T
        w0 = from_f32<BF16>(f16_to_f32(s0) * (float)c0);
        w1 = from_f32<BF16>(f16_to_f32(s1) * (float)c1);
    } else {
        // scale*code + min is exact in f64 (q4/mod.rs:146-147)
        const double v0 = (double)f16_to_f32(s0) * (double)c0 + (double)f16_to_f32(m0);
        const double v1 = (double)f16_to_f32(s1) * (double)c1 + (double)f16_to_f32(m1);
        w0 = BF16 ? f32_to_bf16((float)v0) : f64_to_f16(v0);
        w1 = BF16 ? f32_to_bf16((float)v1) : f64_to_f16(v1);
    }
    return (uint32_t)w0 | ((uint32_t)w1 << 16);
}

template <bool BF16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t w, float acc) {
    if (!BF16) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                      __builtin_bit_cast(half2_t, w), acc, false);
    } else {
        // bf16 x bf16 products are exact in f32; two separately rounded adds
        const float p0 = bf16_to_f32((uint16_t)a) * bf16_to_f32((uint16_t)w);
        const float p1 = bf16_to_f32((uint16_t)(a >> 16)) * bf16_to_f32((uint16_t)(w >> 16));
        return (acc + p0) + p1;
    }
}

template <int M, bool BF16, bool AFFINE>
__global__ void __launch_bounds__(256) q4_gemv_kernel(Q4GemvArgs g, EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *a_lds = (uint16_t *)smem;  // [M][PASS_D]
    float *red = (float *)smem;           // reused at the end: [KL][M][TN]

    const int t = threadIdx.x;
    const int c = t % TN;
    const int kl = t / TN;
    const uint32_t tile = xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t j = tile * TN + c;  // < n_pad always
    const uint32_t block = 1u << g.block_shift;
    const uint32_t last = g.nchunks - 1;

    float acc[M];
#pragma unroll
    for (int r = 0; r < M; r++) acc[r] = 0.0f;

    const uint32_t npass = (g.nchunks + PASS_CH - 1) / PASS_CH;
    for (uint32_t pass = 0; pass < npass; pass++) {
        const uint32_t kc0 = pass * PASS_CH;
        // 0. A[:, pass] into registers first (vmcnt retires in issue order)
        const uint32_t d0 = kc0 * Q4_CHUNK;
        const rsrc_t ar = make_rsrc(g.lhs, g.m * g.k * 2u);
        const bool vec = (g.k & 7) == 0;
        uint4 areg[2 * M];  // element group t + 256*i: row (t + 256 i) / 512
#pragma unroll
        for (int i = 0; i < 2 * M; i++) {
            const uint32_t idx = t + 256 * i;
            areg[i] = load_row8(ar, idx / 512, g.m, g.k, d0 + (idx % 512) * 8, vec);
        }
        // 1. weight loads for the whole pass, branch-free so they overlap
        uint4 wq[P];
        uint16_t sv[P], mv[P];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const uint32_t kc = kc0 + kl * P + p;
            const uint32_t kcc = kc < last ? kc : last;
            wq[p] = *(const uint4 *)(g.nib + cell_index(kcc, j, g.nchunks, g.n_pad) * 16);
            const uint32_t kb = block >= Q4_CHUNK ? ((kcc * Q4_CHUNK) >> g.block_shift) : 0;
            sv[p] = g.sc[cell_index(kb, j, g.sc_rows, g.n_pad)];
            mv[p] = AFFINE ? g.mn[cell_index(kb, j, g.sc_rows, g.n_pad)] : (uint16_t)0;
        }
        // 2. stage A[:, pass] into LDS (zero beyond k)
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2 * M; i++) {
            const uint32_t idx = t + 256 * i;
            *(uint4 *)(a_lds + (idx / 512) * PASS_D + (idx % 512) * 8) = areg[i];
        }
        __syncthreads();
        // 3. dequant + dot
#pragma unroll
        for (int p = 0; p < P; p++) {
            const uint32_t kc = kc0 + kl * P + p;
            if (kc >= g.nchunks) break;
            const uint32_t kcl = kl * P + p;  // chunk within pass
            const uint32_t words[4] = {wq[p].x, wq[p].y, wq[p].z, wq[p].w};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint4 av[M];
#pragma unroll
                for (int r = 0; r < M; r++)
                    av[r] = *(const uint4 *)(a_lds + r * PASS_D + kcl * Q4_CHUNK + w * 8);
                const uint32_t q = words[w];  // stored nibbles are code + 8
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t u = (q >> (4 * e)) & 0x000F000Fu;
                    const int c0 = (int)(u & 0xF) - 8;
                    const int c1 = (int)(u >> 16) - 8;
                    const uint32_t dp = kc * Q4_CHUNK + w * 8 + 2 * e;  // depth of c0
                    uint16_t s0 = sv[p], s1 = sv[p], m0 = mv[p], m1 = mv[p];
                    if (block < Q4_CHUNK) {
                        const uint32_t b0 = dp >> g.block_shift, b1 = (dp + 1) >> g.block_shift;
                        s0 = g.sc[cell_index(b0, j, g.sc_rows, g.n_pad)];
                        s1 = g.sc[cell_index(b1, j, g.sc_rows, g.n_pad)];
                        if (AFFINE) {
                            m0 = g.mn[cell_index(b0, j, g.sc_rows, g.n_pad)];
                            m1 = g.mn[cell_index(b1, j, g.sc_rows, g.n_pad)];
                        }
                    }
                    const uint32_t wpair = deq_pair_generic<BF16, AFFINE>(c0, c1, s0, s1, m0, m1);
#pragma unroll
                    for (int r = 0; r < M; r++) {
                        const uint32_t a2 = e == 0 ? av[r].x : e == 1 ? av[r].y : e == 2 ? av[r].z : av[r].w;
                        acc[r] = dot2<BF16>(a2, wpair, acc[r]);
                    }
                }
            }
        }
    }
    // 4. reduce the KL partial sums of each column in a fixed order
    __syncthreads();
#pragma unroll
    for (int r = 0; r < M; r++) red[(kl * M + r) * TN + c] = acc[r];
    __syncthreads();
    if (t < M * TN) {
        const int r = t / TN, cc = t % TN;
        const uint32_t jj = tile * TN + cc;
        float total = 0.0f;
#pragma unroll
        for (int q = 0; q < KL; q++) total = total + red[(q * M + r) * TN + cc];
        if (r < (int)g.m && jj < g.n)
            g.dst[(size_t)r * g.n + jj] = finish<BF16>(ep, total, r, jj, g.n);
    }
}

template <int M, bool BF16, bool AFFINE>
hipError_t launch_generic(const Q4GemvArgs &g, const EpArgs &ep, hipStream_t s) {
    size_t lds = (size_t)M * PASS_D * 2;
    const size_t red = (size_t)KL * M * TN * 4;
    if (red > lds) lds = red;
    hipLaunchKernelGGL((q4_gemv_kernel<M, BF16, AFFINE>), dim3(g.n_pad / TN), dim3(256), lds, s,
                       g, ep);
    return hipGetLastError();
}

template <int M>
hipError_t launch_variant(const Q4GemvArgs &g, const EpArgs &ep, bool bf16, bool affine,
                          hipStream_t s) {
    if (!bf16 && !affine) return launch_generic<M, false, false>(g, ep, s);
    if (!bf16) return launch_generic<M, false, true>(g, ep, s);
    if (!affine) return launch_generic<M, true, false>(g, ep, s);
    return launch_generic<M, true, true>(g, ep, s);
}

template <int MR, bool CHAIN = false, bool BF16 = false, bool AFFINE = false>
hipError_t launch_mfma(const Q4GemvArgs &g, const EpArgs &ep, hipStream_t s, const ChainArgs &ch = {}) {
    constexpr size_t lds = q4_mfma_lds_bytes<MR, (MR > 8 ? 2 : MF_U)>();
    hipLaunchKernelGGL((q4_gemv_mfma<MR, CHAIN, BF16, AFFINE>), dim3(g.n_pad / 16), dim3(MF_WAVES * 64), lds, s,
                       g, ep, ch);
    return hipGetLastError();
}

template <int MR, bool BF16, bool AFFINE>
hipError_t launch_wave(const Q4GemvArgs &g, const EpArgs &ep, hipStream_t s) {
    constexpr size_t lds = (size_t)MF_WAVES * MR * 1024 + (size_t)MF_WAVES * 16 * MR * 4;
    if (lds > 65536) {
        static bool attr_set = false;  // benign race: every setter writes the same value
        if (!attr_set) {
            const hipError_t e = hipFuncSetAttribute((const void *)q4_gemv_wave<MR, BF16, AFFINE>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
            attr_set = true;
        }
    }
    const uint32_t tiles = g.n_pad / 16;
    hipLaunchKernelGGL((q4_gemv_wave<MR, BF16, AFFINE>), dim3(tiles), dim3(MF_WAVES * 64), lds, s, g.nib, g.sc,
                       g.lhs, g.dst, g.n_pad, g.nchunks, g.k, g.n, tiles, g.m | (ep.n_nodes << 8), g.mn, ep);
    return hipGetLastError();
}

template <bool BF16, bool AFFINE>
hipError_t launch_mfma_rows(const Q4GemvArgs &g, size_t m, const EpArgs &ep, hipStream_t s) {
    // the wave-staged kernel: block 32, 16-byte activation rows, grids it
    // addresses with 32-bit buffer offsets
    if (g.block_shift != 5 || (g.k & 7) != 0 || cell_grid_rows(g.nchunks) * (size_t)g.n_pad * 16 >= ((size_t)1 << 31)) {
        if (m <= 1) return launch_mfma<1, false, BF16, AFFINE>(g, ep, s);
        if (m <= 2) return launch_mfma<2, false, BF16, AFFINE>(g, ep, s);
        if (m <= 4) return launch_mfma<4, false, BF16, AFFINE>(g, ep, s);
        if (m <= 8) return launch_mfma<8, false, BF16, AFFINE>(g, ep, s);
        return launch_mfma<16, false, BF16, AFFINE>(g, ep, s);
    }
    if (m <= 1) return launch_wave<1, BF16, AFFINE>(g, ep, s);
    if (m <= 2) return launch_wave<2, BF16, AFFINE>(g, ep, s);
    if (m <= 4) return launch_wave<4, BF16, AFFINE>(g, ep, s);
    if (m <= 8) return launch_wave<8, BF16, AFFINE>(g, ep, s);
    return launch_wave<16, BF16, AFFINE>(g, ep, s);
}


}  // namespace

hipError_t launch_q4_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                          const EpArgs &ep, bool bf16, hipStream_t s) {
    if (!q4_gemv_serves(w, m)) return hipErrorNotSupported;
    const Q4GemvArgs g = q4_gemv_args(w, m, dst, lhs);
    const bool affine = w.mins != nullptr;
    if ((size_t)m * w.k * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;  // buffer range
    if (w.nchunks == 0) {
        // k == 0: every product is the empty sum; the generic kernel runs no
        // pass and stores ep(+0)
        if (m <= 1) return launch_generic<1, false, false>(g, ep, s);
        return launch_generic<8, false, false>(g, ep, s);
    }
    if (w.block >= (size_t)Q4_CHUNK) {  // one scale (and min) per chunk: the matrix-core GEMV
        if (!bf16 && !affine) return launch_mfma_rows<false, false>(g, m, ep, s);
        if (!bf16) return launch_mfma_rows<false, true>(g, m, ep, s);
        if (!affine) return launch_mfma_rows<true, false>(g, m, ep, s);
        return launch_mfma_rows<true, true>(g, m, ep, s);
    }
    if (m <= 1) return launch_variant<1>(g, ep, bf16, affine, s);
    if (m <= 2) return launch_variant<2>(g, ep, bf16, affine, s);
    if (m <= 4) return launch_variant<4>(g, ep, bf16, affine, s);
    return launch_variant<8>(g, ep, bf16, affine, s);
}

hipError_t launch_q4_gemv_chained(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                                  const EpArgs &ep, const ChainArgs &ch, hipStream_t s) {
    if (m < 1 || m > Q4_GEMV_MAX_ROWS || w.mins != nullptr || w.block < (size_t)Q4_CHUNK || w.nchunks == 0)
        return hipErrorNotSupported;
    if ((size_t)m * w.k * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;  // buffer range
    const Q4GemvArgs g = q4_gemv_args(w, m, dst, lhs);
    if (m <= 1) return launch_mfma<1, true>(g, ep, s, ch);
    if (m <= 2) return launch_mfma<2, true>(g, ep, s, ch);
    if (m <= 4) return launch_mfma<4, true>(g, ep, s, ch);
    return launch_mfma<8, true>(g, ep, s, ch);
}

}  // namespace smg
