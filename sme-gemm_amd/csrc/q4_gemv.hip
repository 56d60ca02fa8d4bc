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
// The call is HBM-bound (0.5625 B of weights per MAC at block 32). Each
// workgroup owns 16 output columns and splits K over 16 lanes; every lane
// issues all of its 16-byte weight loads for a 4096-depth pass before it
// touches A, so a whole pass of the weight matrix is in flight at once. A
// (<= 64 KB) is staged in LDS per pass and read with broadcast ds_read_b128.
#include "kernels.h"

namespace smg {

namespace {

constexpr int TN = 16;        // output columns per workgroup
constexpr int KL = 16;        // lanes along K per column
constexpr int P = 8;          // chunks per lane per pass
constexpr int PASS_CH = KL * P;            // chunks per pass
constexpr int PASS_D = PASS_CH * Q4_CHUNK; // depths per pass (4096)

struct Q4GemvArgs {
    const uint8_t *nib;
    const uint16_t *sc;
    const uint16_t *mn;
    const uint16_t *lhs;
    uint16_t *dst;
    uint32_t n, k, n_pad, nchunks, m;
    uint32_t block_shift;  // log2(block)
};

// Two consecutive depths' weights as a packed pair of 16-bit values.
// Generic form: any block size, affine or not, f16 or bf16 (the exact
// reference roundings, computed per value).
template <bool BF16, bool AFFINE>
__device__ __forceinline__ uint32_t deq_pair_generic(int c0, int c1, uint16_t s0, uint16_t s1,
                                                     uint16_t m0, uint16_t m1) {
    uint16_t w0, w1;
    if (!AFFINE) {
        // scale*code is exact in f32 (11-bit x 4-bit), so one rounding to T
        float v0 = f16_to_f32(s0) * (float)c0;
        float v1 = f16_to_f32(s1) * (float)c1;
        w0 = from_f32<BF16>(v0);
        w1 = from_f32<BF16>(v1);
    } else {
        // scale*code + min is exact in f64 (q4/mod.rs:146-147)
        double v0 = (double)f16_to_f32(s0) * (double)c0 + (double)f16_to_f32(m0);
        double v1 = (double)f16_to_f32(s1) * (double)c1 + (double)f16_to_f32(m1);
        if (BF16) {
            w0 = f32_to_bf16((float)v0);
            w1 = f32_to_bf16((float)v1);
        } else {
            w0 = f64_to_f16(v0);
            w1 = f64_to_f16(v1);
        }
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
        float p0 = bf16_to_f32((uint16_t)a) * bf16_to_f32((uint16_t)w);
        float p1 = bf16_to_f32((uint16_t)(a >> 16)) * bf16_to_f32((uint16_t)(w >> 16));
        return (acc + p0) + p1;
    }
}

// FAST: f16, scale-only, block >= 32 (one scale per chunk): the nibble pair
// (code+8 after the xor) becomes 1024+u in f16, minus 1032 gives the exact
// code, and one packed f16 multiply by the scale is the reference's single
// RNE rounding of scale*code.
template <int M, bool BF16, bool AFFINE, bool FAST>
__global__ void __launch_bounds__(256) q4_gemv_kernel(Q4GemvArgs g, EpArgs ep) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *a_lds = (uint16_t *)smem;  // [M][PASS_D]
    float *red = (float *)smem;           // reused at the end: [KL][M][TN]

    const int t = threadIdx.x;
    const int c = t % TN;
    const int kl = t / TN;
    const uint32_t j = blockIdx.x * TN + c;  // < n_pad always
    const uint32_t block = 1u << g.block_shift;

    float acc[M];
#pragma unroll
    for (int r = 0; r < M; r++) acc[r] = 0.0f;

    const uint32_t npass = (g.nchunks + PASS_CH - 1) / PASS_CH;
    for (uint32_t pass = 0; pass < npass; pass++) {
        const uint32_t kc0 = pass * PASS_CH;
        // 1. weight loads for the whole pass, issued before anything waits
        uint4 wq[P];
        uint16_t sv[P];
        uint16_t mv[P];
#pragma unroll
        for (int p = 0; p < P; p++) {
            uint32_t kc = kc0 + kl * P + p;
            if (kc < g.nchunks) {
                wq[p] = *(const uint4 *)(g.nib + ((size_t)kc * g.n_pad + j) * 16);
                if (FAST || block >= Q4_CHUNK) {
                    uint32_t kb = (kc * Q4_CHUNK) >> g.block_shift;
                    sv[p] = g.sc[(size_t)kb * g.n_pad + j];
                    if (AFFINE) mv[p] = g.mn[(size_t)kb * g.n_pad + j];
                }
            } else {
                wq[p] = make_uint4(0, 0, 0, 0);
                sv[p] = 0;
                mv[p] = 0;
            }
        }
        // 2. stage A[:, pass] into LDS (zero beyond k)
        __syncthreads();
        const uint32_t d0 = kc0 * Q4_CHUNK;
        for (uint32_t idx = t; idx < (uint32_t)M * PASS_D / 8; idx += 256) {
            uint32_t r = idx / (PASS_D / 8);
            uint32_t x = (idx % (PASS_D / 8)) * 8;
            uint32_t d = d0 + x;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (r < g.m) {
                const uint16_t *src = g.lhs + (size_t)r * g.k + d;
                if (d + 8 <= g.k && ((((uintptr_t)src) & 15) == 0)) {
                    v = *(const uint4 *)src;
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int q = 0; q < 8; q++) e[q] = (d + q < g.k) ? src[q] : (uint16_t)0;
                    v.x = e[0] | ((uint32_t)e[1] << 16);
                    v.y = e[2] | ((uint32_t)e[3] << 16);
                    v.z = e[4] | ((uint32_t)e[5] << 16);
                    v.w = e[6] | ((uint32_t)e[7] << 16);
                }
            }
            *(uint4 *)(a_lds + r * PASS_D + x) = v;
        }
        __syncthreads();
        // 3. dequant + dot
#pragma unroll
        for (int p = 0; p < P; p++) {
            uint32_t kc = kc0 + kl * P + p;
            if (kc >= g.nchunks) break;
            const uint32_t kcl = kl * P + p;  // chunk within pass
            uint32_t words[4] = {wq[p].x, wq[p].y, wq[p].z, wq[p].w};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint4 av[M];
#pragma unroll
                for (int r = 0; r < M; r++)
                    av[r] = *(const uint4 *)(a_lds + r * PASS_D + kcl * Q4_CHUNK + w * 8);
                uint32_t q = words[w] ^ 0x88888888u;  // nibble -> code + 8
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t u = (q >> (4 * e)) & 0x000F000Fu;
                    uint32_t wpair;
                    if (FAST) {
                        half2_t h = __builtin_bit_cast(half2_t, u | 0x64006400u);
                        const half2_t magic = {(_Float16)1032.0f, (_Float16)1032.0f};
                        _Float16 s = __builtin_bit_cast(_Float16, sv[p]);
                        half2_t s2 = {s, s};
                        half2_t wv = (h - magic) * s2;
                        wpair = __builtin_bit_cast(uint32_t, wv);
                    } else {
                        int c0 = (int)(u & 0xF) - 8;
                        int c1 = (int)(u >> 16) - 8;
                        uint32_t dp = kc * Q4_CHUNK + w * 8 + 2 * e;  // depth of c0
                        uint16_t s0, s1, m0 = 0, m1 = 0;
                        if (block >= Q4_CHUNK) {
                            s0 = s1 = sv[p];
                            if (AFFINE) m0 = m1 = mv[p];
                        } else {
                            uint32_t b0 = dp >> g.block_shift, b1 = (dp + 1) >> g.block_shift;
                            s0 = g.sc[(size_t)b0 * g.n_pad + j];
                            s1 = g.sc[(size_t)b1 * g.n_pad + j];
                            if (AFFINE) {
                                m0 = g.mn[(size_t)b0 * g.n_pad + j];
                                m1 = g.mn[(size_t)b1 * g.n_pad + j];
                            }
                        }
                        wpair = deq_pair_generic<BF16, AFFINE>(c0, c1, s0, s1, m0, m1);
                    }
#pragma unroll
                    for (int r = 0; r < M; r++) {
                        uint32_t a2 = e == 0 ? av[r].x : e == 1 ? av[r].y : e == 2 ? av[r].z : av[r].w;
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
        const uint32_t jj = blockIdx.x * TN + cc;
        float total = 0.0f;
#pragma unroll
        for (int q = 0; q < KL; q++) total = total + red[(q * M + r) * TN + cc];
        if (r < (int)g.m && jj < g.n)
            g.dst[(size_t)r * g.n + jj] = finish<BF16>(ep, total, r, jj, g.n);
    }
}

template <int M, bool BF16, bool AFFINE, bool FAST>
hipError_t launch_m(const Q4GemvArgs &g, const EpArgs &ep, hipStream_t s) {
    size_t lds = (size_t)M * PASS_D * 2;
    size_t red = (size_t)KL * M * TN * 4;
    if (red > lds) lds = red;
    dim3 grid(g.n_pad / TN);
    hipLaunchKernelGGL((q4_gemv_kernel<M, BF16, AFFINE, FAST>), grid, dim3(256), lds, s, g, ep);
    return hipGetLastError();
}

template <int M>
hipError_t launch_variant(const Q4GemvArgs &g, const EpArgs &ep, bool bf16, bool affine,
                          bool big_block, hipStream_t s) {
    if (!bf16 && !affine && big_block) return launch_m<M, false, false, true>(g, ep, s);
    if (!bf16 && !affine) return launch_m<M, false, false, false>(g, ep, s);
    if (!bf16) return launch_m<M, false, true, false>(g, ep, s);
    if (!affine) return launch_m<M, true, false, false>(g, ep, s);
    return launch_m<M, true, true, false>(g, ep, s);
}

}  // namespace

hipError_t launch_q4_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                          const EpArgs &ep, bool bf16, hipStream_t s) {
    Q4GemvArgs g;
    g.nib = w.codes;
    g.sc = w.scales;
    g.mn = w.mins;
    g.lhs = lhs;
    g.dst = dst;
    g.n = (uint32_t)w.n;
    g.k = (uint32_t)w.k;
    g.n_pad = (uint32_t)w.n_pad;
    g.nchunks = (uint32_t)w.nchunks;
    g.m = (uint32_t)m;
    g.block_shift = (uint32_t)__builtin_ctzll(w.block);
    const bool affine = w.mins != nullptr;
    const bool big = w.block >= (size_t)Q4_CHUNK;
    if (m <= 1) return launch_variant<1>(g, ep, bf16, affine, big, s);
    if (m <= 2) return launch_variant<2>(g, ep, bf16, affine, big, s);
    if (m <= 4) return launch_variant<4>(g, ep, bf16, affine, big, s);
    return launch_variant<8>(g, ep, bf16, affine, big, s);
}

}  // namespace smg
