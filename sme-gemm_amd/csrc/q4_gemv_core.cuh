// The main loop of the Q4 MFMA GEMV (decode-shaped m <= 8), shared by the plain
// GEMV (q4_gemv.hip) and the decode block's fused kernels (decode_block.hip),
// which differ only in where the activation rows come from (an f16 array, or
// an RMS-normalized f32 residual row) and in what their stores do.
//
// A workgroup of 8 waves owns 16 output columns; wave w takes every 8th group
// of 4 chunks (128 depths). Lane (g = lane/16, c = lane%16) loads the 16-byte
// chunk g of column c, so a wave load reads one contiguous 1 KB run of the
// blocked layout (common.cuh), and every lane issues all its weight loads before it
// waits. Each dword (8
// depths) dequantizes to 8 f16 weights -- v_bfi_b32 puts the nibble under an
// f16 exponent, a packed subtract leaves the exact code, a packed multiply by
// the scale is the reference's single RNE rounding of scale*code -- and feeds
// one v_mfma_f32_16x16x32_f16 as the A operand (16 columns x 32 depths), with
// up to 16 activation rows as the B operand.
#pragma once

#include "kernels.h"

namespace smg {

struct Q4GemvArgs {
    const uint8_t *nib;
    const uint16_t *sc;
    const uint16_t *mn;
    const uint16_t *lhs;
    uint16_t *dst;
    uint32_t n, k, n_pad, nchunks, m;
    uint32_t sc_rows;      // rows of the scale (and min) grids
    uint32_t block_shift;  // log2(block)
};

constexpr int MF_WAVES = 8;                  // waves per workgroup (K slices)
constexpr int MF_U = 4;                      // steps (4 chunks each) in flight per lane
constexpr int MF_SEG = 4096;                 // depths of A staged in LDS at a time
constexpr int MF_SEG_CH = MF_SEG / Q4_CHUNK; // 128 chunks per segment

// One wait of a chained call (thread 0 of the workgroup): polls *ready until it
// reaches need or the device wall clock has advanced `ticks` (and at most 2^24
// polls), then an agent-scope acquire, so the producer's stores of A below
// need are visible to the loads that follow the workgroup barrier.
__device__ __forceinline__ bool chain_wait(const unsigned long long *ready, unsigned long long need,
                                           unsigned long long ticks) {
    const unsigned long long t0 = wall_clock64();
    for (uint32_t it = 0; it < (1u << 24); it++) {
        if (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= need) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            return true;
        }
        if (wall_clock64() - t0 > ticks) break;
        __builtin_amdgcn_s_sleep(4);
    }
    return false;
}

// Activation source: MR rows of a row-major f16 [m][k] array (rows >= m and
// depths >= k read as zero, through buffer loads with no branches).
// A source loads thread t's share of a segment (`load`, issued before the
// weight loads) into its Regs and writes the segment's f16 rows to LDS
// (`stage`, all threads, between two barriers).
template <int MR, int SEG = MF_SEG>
struct SrcRows {
    static constexpr int SEG_D = SEG;  // depths staged per segment (the LDS row stride)
    struct Regs {
        uint4 r[MR];
    };
    rsrc_t ar;
    uint32_t m, k;
    bool vec;
    __device__ SrcRows(const uint16_t *lhs, uint32_t m_, uint32_t k_)
        : ar(make_rsrc(lhs, m_ * k_ * 2u)), m(m_), k(k_), vec((k_ & 7) == 0) {}
    // thread t's 8 depths d0 + 8t .. +8 of every row (threads past the
    // segment load and stage nothing)
    static constexpr bool ALL = SEG >= 8 * MF_WAVES * 64;  // every thread has depths of the segment
    __device__ void load(Regs &a, uint32_t d0, int t) const {
#pragma unroll
        for (int r = 0; r < MR; r++)
            a.r[r] = ALL || 8 * t < SEG ? load_row8(ar, r, m, k, d0 + 8 * t, vec) : make_uint4(0, 0, 0, 0);
    }
    __device__ void stage(uint16_t *a_lds, const Regs &a, int t) const {
#pragma unroll
        for (int r = 0; r < MR; r++)
            if (ALL || 8 * t < SEG) *(uint4 *)(a_lds + r * SEG + 8 * t) = a.r[r];
    }
};

// The workgroup's accumulator tile for 16 columns (col = tile*16 + lane%16):
// lane holds D[col = 4*(lane/16) + v][row = lane%16] of its wave's K slice.
// CHAIN: the chained GEMV's wait for its producer (ch.ready) between the weight
// loads and the activation loads of each segment; timed_out reports a wait
// that expired (uniform over the workgroup; the tile is then incomplete).
// MASK_B: only the B lanes of rows < MR read LDS, under an exec mask, the
// others zeroed; otherwise every lane reads (rows >= MR read row MR-1 again:
// MFMA output rows are independent and those are never read). Measured on
// MI355X, masking is 0.18 us faster for the lone config-1 GEMV from HBM, and
// reading everywhere 1.7 us faster over a decode step's five projections,
// whose wide GEMVs are bound by the VALU the zeroing adds.
// BF16: bf16 activations and weights (v_mfma_f32_16x16x32_bf16; each weight
// bf16_RNE(f32(scale) * code [+ f32(min)]), q4_deq8_bf16); AFFINE: Q4_1
// weights with their mins (f16: q4_deq8_affine).
// U: steps per lane per segment (a segment is U * 1024 depths; Src::SEG_D
// must match): 4, or 2 for 16 rows, whose staged segment then fits 64 KB.
template <int MR, bool CHAIN, class Src, bool MASK_B = true, bool BF16 = false, bool AFFINE = false,
          int U = MF_U>
__device__ __forceinline__ float4_t q4_mfma_mainloop(const Q4GemvArgs &g, const Src &src,
                                                     const ChainArgs &ch, uint16_t *a_lds, uint32_t col,
                                                     bool &timed_out) {
    constexpr int SEG_CH = 4 * MF_WAVES * U;  // chunks per segment
    constexpr int SEG = SEG_CH * Q4_CHUNK;    // depths per segment
    static_assert(SEG == Src::SEG_D, "the source stages the segment the loop multiplies");
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int c = lane & 15, grp = lane >> 4;
    // the bfi magics live in VGPRs (a VOP3 takes one scalar operand)
    const uint32_t mag_lo = __builtin_amdgcn_readfirstlane(0x64006400u) | (uint32_t)(t >> 30);
    const uint32_t mag_hi = __builtin_amdgcn_readfirstlane(0x54005400u) | (uint32_t)(t >> 30);
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    timed_out = false;
    const uint32_t last = g.nchunks - 1;  // nchunks >= 1 here
    const uint32_t nseg = (g.nchunks + SEG_CH - 1) / SEG_CH;
    for (uint32_t seg = 0; seg < nseg; seg++) {
        const uint32_t sc0 = seg * SEG_CH;
        // A[:, segment] first: vmcnt retires in issue order, so loads issued
        // before the weights can be waited on while the weights stay in flight
        const uint32_t d0 = sc0 * Q4_CHUNK;
        typename Src::Regs areg;
        bool a_first = true;  // a chained call that awaits A reads it after its weights
        if constexpr (CHAIN) a_first = ch.ready == nullptr;
        if (a_first) src.load(areg, d0, t);
        // steps of this wave within the segment: chunks sc0 + 4*(wave + 8*u) + grp
        uint4 wq[U];
        uint16_t sv[U], mv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t kc = sc0 + 4 * (wave + MF_WAVES * u) + grp;
            const uint32_t kcc = kc < last ? kc : last;  // clamped: always a valid load
            wq[u] = *(const uint4 *)(g.nib + cell_index(kcc, col, g.nchunks, g.n_pad) * 16);
            const size_t si = cell_index((kcc * Q4_CHUNK) >> g.block_shift, col, g.sc_rows, g.n_pad);
            const uint16_t sl = g.sc[si];
            sv[u] = kc < g.nchunks ? sl : (uint16_t)0;  // a dead step's weights become 0
            if constexpr (AFFINE) {
                const uint16_t ml = g.mn[si];
                mv[u] = kc < g.nchunks ? ml : (uint16_t)0;
            }
        }
        if constexpr (CHAIN) {
            // the weights stream in while the producer of A finishes; A's
            // segment is read only once *ready covers it
            if (ch.ready) {
                __shared__ uint32_t seg_ok;
                if (t == 0) {
                    const uint32_t need = g.k < d0 + SEG ? g.k : d0 + SEG;
                    seg_ok = chain_wait(ch.ready, need, ch.wait_ticks) ? 1u : 0u;
                }
                __syncthreads();
                if (!seg_ok) {
                    timed_out = true;
                    break;
                }
                src.load(areg, d0, t);
            }
        }
        // stage A[:, segment] (rows < m, zero past k)
        __syncthreads();
        src.stage(a_lds, areg, t);
        __syncthreads();
        // dequant + MFMA: A operand = 16 columns x 32 depths of weights, B
        // operand = 32 depths x 16 rows of activations (B lanes per MASK_B).
        // Chunks past K read the staged zeros of the segment and have zero
        // weights. All of this wave's activation fragments are read first, so
        // the LDS round trips overlap instead of each one preceding its MFMA.
        const uint16_t *arow = a_lds + (c < MR ? c : MR - 1) * SEG;
        uint4 abv[U][4];
        if (!MASK_B || c < MR) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint32_t kcl = 4 * (wave + MF_WAVES * u) + grp;  // chunk within the segment
#pragma unroll
                for (int w = 0; w < 4; w++) abv[u][w] = *(const uint4 *)(arow + kcl * Q4_CHUNK + w * 8);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int w = 0; w < 4; w++) abv[u][w] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const half2_t s2 = {__builtin_bit_cast(_Float16, sv[u]), __builtin_bit_cast(_Float16, sv[u])};
            const uint32_t words[4] = {wq[u].x, wq[u].y, wq[u].z, wq[u].w};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                if constexpr (BF16) {
                    const uint32_t s1 = sv[u];
                    const float mf = AFFINE ? f16_to_f32(mv[u]) : -0.0f;
                    const uint4 wa = q4_deq8_bf16(words[w], s1, mf, mag_lo, mag_hi);
                    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wa),
                                                                  __builtin_bit_cast(bf16x8_t, abv[u][w]), acc,
                                                                  0, 0, 0);
                } else {
                    uint4 wa;
                    if constexpr (AFFINE) {
                        const half2_t m2 = {__builtin_bit_cast(_Float16, mv[u]), __builtin_bit_cast(_Float16, mv[u])};
                        wa = q4_deq8_affine(words[w], s2, m2, mag_lo, mag_hi);
                    } else {
                        wa = q4_deq8(words[w], s2, mag_lo, mag_hi);
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, wa),
                                                                 __builtin_bit_cast(half8_t, abv[u][w]), acc,
                                                                 0, 0, 0);
                }
            }
        }
    }
    return acc;
}

// One item of a persistent single-row GEMV (a workgroup that walks several
// tiles): this lane's MF_U weight chunks of segment sc0 for column col, with
// their scales, loaded before the previous item is multiplied so one item's
// loads are always in flight behind the MFMAs. Past the last chunk the load
// is clamped to a valid address and the scale is zero, as in the main loop.
struct Q4Item {
    uint4 wq[MF_U];
    uint32_t sv[MF_U];
};
__device__ __forceinline__ void q4_item_load(const Q4GemvArgs &g, uint32_t sc0, uint32_t col, Q4Item &it) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = lane >> 4;
    const uint32_t last = g.nchunks - 1;
#pragma unroll
    for (int u = 0; u < MF_U; u++) {
        const uint32_t kc = sc0 + 4 * (wave + MF_WAVES * u) + grp;
        const uint32_t kcc = kc < last ? kc : last;
        it.wq[u] = *(const uint4 *)(g.nib + cell_index(kcc, col, g.nchunks, g.n_pad) * 16);
        const uint16_t sl = g.sc[cell_index((kcc * Q4_CHUNK) >> g.block_shift, col, g.sc_rows, g.n_pad)];
        it.sv[u] = kc < g.nchunks ? sl : 0u;
    }
}
// The item's MFMAs for activation row 0, staged in LDS at arow[depth] (the
// whole row, zero-filled to whole segments): every B-operand lane reads row 0
// (q4_mfma_mainloop's unmasked form), and only output row 0 is used.
__device__ __forceinline__ void q4_item_mma1(uint32_t sc0, const Q4Item &it, const uint16_t *arow,
                                             float4_t &acc, uint32_t mag_lo, uint32_t mag_hi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 4;
#pragma unroll
    for (int u = 0; u < MF_U; u++) {
        const uint32_t kc = sc0 + 4 * (wave + MF_WAVES * u) + grp;
        uint4 ab[4];
#pragma unroll
        for (int w = 0; w < 4; w++) ab[w] = *(const uint4 *)(arow + kc * Q4_CHUNK + w * 8);
        const half2_t s2 = {__builtin_bit_cast(_Float16, (uint16_t)it.sv[u]),
                            __builtin_bit_cast(_Float16, (uint16_t)it.sv[u])};
        const uint32_t words[4] = {it.wq[u].x, it.wq[u].y, it.wq[u].z, it.wq[u].w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint4 wa = q4_deq8(words[w], s2, mag_lo, mag_hi);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, wa),
                                                         __builtin_bit_cast(half8_t, ab[w]), acc, 0, 0, 0);
        }
    }
}

// The 8 waves' partial tiles into red[MF_WAVES][16 cols][MR] (LDS, after a
// barrier; a_lds may alias red), then a barrier: afterwards tile_total(red,
// cc, r) is column cc's (0..15) sum for row r, in a fixed wave order.
template <int MR>
__device__ __forceinline__ void q4_mfma_reduce(const float4_t &acc, float *red) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int c = lane & 15, grp = lane >> 4;
    __syncthreads();
    if (c < MR) {
#pragma unroll
        for (int v = 0; v < 4; v++) red[(wave * 16 + 4 * grp + v) * MR + c] = acc[v];
    }
    __syncthreads();
}
template <int MR>
__device__ __forceinline__ float tile_total(const float *red, int cc, int r) {
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < MF_WAVES; w++) total = total + red[(w * 16 + cc) * MR + r];
    return total;
}

// ---------------------------------------------------------------------------
// Wave-staged main loop (the plain GEMV's): the same 8 waves x 16 columns and
// the same per-lane chunks as q4_mfma_mainloop, but each wave stages only the
// activations its own chunks multiply -- wave w's chunks of a 4096-depth
// segment are the four 128-depth runs at (seg*128 + 4*(w + 8u)) * 32, u = 0..3,
// 256 bytes a row each -- into a 1 KB-a-row region of LDS that no other wave
// reads. So no workgroup barrier separates a wave's activation loads from its
// MFMAs: a wave starts as soon as its own bytes arrive (LDS operations of one
// wave execute in order, so its reads see its writes). One load per lane and
// row covers the wave's 1 KB: lane L loads 8 depths of run L/16 at offset
// (L%16)*8, and writes them to LDS at L*16 bytes.
// ---------------------------------------------------------------------------
struct Q4WaveArgs {
    rsrc_t nr, sr, mr;    // nibble / scale / min grids (byte counts under 2^31; past them reads 0)
    rsrc_t ar;            // activation rows [m][k], k a multiple of 8 (zero outside)
    uint32_t n_pad, nchunks, k, m;
};

// One 4096-depth segment of the wave-staged loop (block 32: one scale cell
// per chunk). Addresses are 32-bit buffer offsets: chunk kc = sc0 +
// 4*(wave + 8u) + grp of column col is cell (kc, col) of the nibble and of the
// scale grid, whose 4-row block index is sc0/4 + wave + 8u, so the four
// steps' offsets differ by the constant 8 blocks (512 * n_pad bytes of
// nibbles, 64 * n_pad of scales).
template <int MR, bool BF16, bool AFFINE>
__device__ __forceinline__ void q4_wave_segment(const Q4WaveArgs &g, uint16_t *wlds, uint32_t col, uint32_t sc0,
                                                uint32_t mag_lo, uint32_t mag_hi, float4_t &acc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, grp = lane >> 4;
    // this wave's activations first (vmcnt retires in issue order)
    uint4 areg[MR];
    const uint32_t da = (sc0 + 4 * (wave + MF_WAVES * grp)) * Q4_CHUNK + (lane & 15) * 8;
#pragma unroll
    for (int r = 0; r < MR; r++) areg[r] = bload16(g.ar, (r < (int)g.m && da < g.k) ? (r * g.k + da) * 2u : OOB);
    const uint32_t cell0 = ((sc0 >> 2) + wave) * 4 * g.n_pad + grp * 16 + (col >> 4) * 64 + (col & 15);
    // each step's nibbles and scale (and min) are issued together, step by
    // step (the scheduling barrier keeps the compiler from hoisting every
    // scale load first): vmcnt retires in issue order, so step 0 can be
    // multiplied as soon as its own bytes land while steps 1-3 stream in
    // (config 1: 3.92 -> 3.77 us a call against scales-first); the streaming
    // cache policy keeps the weights from displacing A and the code in L2
    uint4 wq[MF_U];
    uint16_t sv[MF_U], mv[MF_U];
#pragma unroll
    for (int u = 0; u < MF_U; u++) {
        const uint32_t kc = sc0 + 4 * (wave + MF_WAVES * u) + grp;
        wq[u] = bload16_nt(g.nr, cell0 * 16 + u * 512 * g.n_pad);
        const uint32_t so = cell0 * 2 + u * 64 * g.n_pad;
        const uint16_t sl = bload2_nt(g.sr, so);
        // a step past K has zero weights (the padding rows of a gathered grid
        // are not written, so its nibbles and scales may hold anything finite
        // or not: only the scale is replaced)
        sv[u] = kc < g.nchunks ? sl : (uint16_t)0;
        if constexpr (AFFINE) {
            const uint16_t ml = bload2_nt(g.mr, so);
            mv[u] = kc < g.nchunks ? ml : (uint16_t)0;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < MR; r++) *(uint4 *)(wlds + r * 512 + lane * 8) = areg[r];
    // fragments: lane (c, grp) reads row c's 8 depths of dword w of chunk
    // grp of run u, at [c][u][grp * 32 + w * 8]
    uint4 abv[MF_U][4];
    if (c < MR) {
#pragma unroll
        for (int u = 0; u < MF_U; u++)
#pragma unroll
            for (int w = 0; w < 4; w++) abv[u][w] = *(const uint4 *)(wlds + c * 512 + u * 128 + grp * 32 + w * 8);
    } else {
#pragma unroll
        for (int u = 0; u < MF_U; u++)
#pragma unroll
            for (int w = 0; w < 4; w++) abv[u][w] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < MF_U; u++) {
        const half2_t s2 = {__builtin_bit_cast(_Float16, sv[u]), __builtin_bit_cast(_Float16, sv[u])};
        const uint32_t words[4] = {wq[u].x, wq[u].y, wq[u].z, wq[u].w};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            if constexpr (BF16) {
                const float mf = AFFINE ? f16_to_f32(mv[u]) : -0.0f;
                const uint4 wa = q4_deq8_bf16(words[w], sv[u], mf, mag_lo, mag_hi);
                typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wa),
                                                              __builtin_bit_cast(bf16x8_t, abv[u][w]), acc, 0, 0, 0);
            } else {
                uint4 wa;
                if constexpr (AFFINE) {
                    const half2_t m2 = {__builtin_bit_cast(_Float16, mv[u]), __builtin_bit_cast(_Float16, mv[u])};
                    wa = q4_deq8_affine(words[w], s2, m2, mag_lo, mag_hi);
                } else {
                    wa = q4_deq8(words[w], s2, mag_lo, mag_hi);
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, wa),
                                                             __builtin_bit_cast(half8_t, abv[u][w]), acc, 0, 0, 0);
            }
        }
    }
}

// The whole of K, segment by segment; the first segment is peeled so that a
// call of K <= 4096 runs straight-line code from the kernel's entry to its
// last MFMA (instruction fetch after a launch reaches far memory).
template <int MR, bool BF16, bool AFFINE>
__device__ __forceinline__ float4_t q4_wave_loop(const Q4WaveArgs &g, uint16_t *wlds, uint32_t col) {
    const int t = threadIdx.x;
    const uint32_t mag_lo = __builtin_amdgcn_readfirstlane(0x64006400u) | (uint32_t)(t >> 30);
    const uint32_t mag_hi = __builtin_amdgcn_readfirstlane(0x54005400u) | (uint32_t)(t >> 30);
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    q4_wave_segment<MR, BF16, AFFINE>(g, wlds, col, 0, mag_lo, mag_hi, acc);
    const uint32_t nseg = (g.nchunks + MF_SEG_CH - 1) / MF_SEG_CH;
    for (uint32_t seg = 1; seg < nseg; seg++)
        q4_wave_segment<MR, BF16, AFFINE>(g, wlds, col, seg * MF_SEG_CH, mag_lo, mag_hi, acc);
    return acc;
}

// LDS bytes of a q4_mfma_mainloop kernel staging MR rows of a U-step segment
// (also covers red).
template <int MR, int U = MF_U>
constexpr size_t q4_mfma_lds_bytes() {
    return (size_t)MR * U * 1024 * 2 > (size_t)MF_WAVES * 16 * MR * 4 ? (size_t)MR * U * 1024 * 2
                                                                       : (size_t)MF_WAVES * 16 * MR * 4;
}

inline Q4GemvArgs q4_gemv_args(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs) {
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
    g.sc_rows = (uint32_t)w.sc_rows;
    g.m = (uint32_t)m;
    g.block_shift = (uint32_t)__builtin_ctzll(w.block);
    return g;
}

}  // namespace smg
