// The decode block (one row through src/block.rs's Block::accumulate) on
// gfx950, with the reference's row-wise passes fused into the kernels that
// need them:
//
//   blk_gemv<NORM, QKV>   RMSNorm of the f32 residual row (src/nn.rs:127-144)
//                         staged as the GEMV's f16 activations, the qkv Q4 GEMV,
//                         and at the store the NeoX RoPE (examples/bonsai/
//                         model.rs:87-99) of q and k, the new key / value row
//                         written into the cache, q rounded after the score
//                         scale as attention_kv_f16 rounds it
//                         (src/kernels/kv_attention.rs:298-302);
//   attn_split            flash-decode partials: per (KV head, chunk of its
//                         query heads, 64-key split) the scores, a local softmax
//                         and its value sums;
//   attn_combine          the splits merged (max-rescaled), / sum, rounded to
//                         f16 for the out projection (or f32 for the API);
//   blk_gemv<.., RESID>   the out / down Q4 GEMV adding its f16-rounded result
//                         into the f32 residual (convert::add_f16, src/convert.rs);
//   blk_gemv<NORM, GLU>   RMSNorm again, the gate/up Q4 GEMV, and GatedLinear's
//                         glu (src/linear.rs:804-826) at the store.
//
// Numerics: every rounding point of the reference is kept (the f16 GEMV
// outputs, q, the cache rows, the attention output, the hidden layer, the
// residual adds); sums run in other orders (split-K GEMV, a tree for the sum
// of squares, split softmax) and exp / tanh are the device's, so results are
// held to a tolerance against the portable path, not to its bits.
#include <atomic>

#include "q4_gemv_core.cuh"

namespace smg {

namespace {

// Cross-lane reductions on DPP (a VALU operand modifier, no LDS round trip):
// within a 16-lane row, quad_perm [1,0,3,2] and [2,3,0,1] pair lanes i ^ 1
// and i ^ 2 (each lane then holds its quad's total), row_half_mirror pairs
// lane i with 7 - i (the other quad of its half row) and row_mirror pairs i
// with 15 - i (the other half row). Each pair adds the same two values, so
// every lane of a group ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int G>  // aligned groups of G lanes, G = 8, 16 or 32
__device__ __forceinline__ float dpp_group_sum(float v) {
    v = v + dppf<0xB1>(v);
    v = v + dppf<0x4E>(v);
    v = v + dppf<0x141>(v);
    if constexpr (G > 8) v = v + dppf<0x140>(v);
    if constexpr (G > 16) v = v + __shfl_xor(v, 16);
    return v;
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dppf<0xB1>(v));
    v = fmaxf(v, dppf<0x4E>(v));
    v = fmaxf(v, dppf<0x141>(v));
    return fmaxf(v, dppf<0x140>(v));
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Over the wave: the four rows' totals read into scalars and combined in
// row order (the result is uniform: every lane holds the same bits).
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_group_sum<16>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ float4 bload16f(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// 1 / sqrt(mean(x^2) + eps) over a workgroup of MF_WAVES waves, from each
// thread's partial sum of squares (fixed combination order: every thread gets
// the same bits). Correctly rounded division and square root (HIP's default).
__device__ __forceinline__ float rms_scale(float ss, uint32_t k, float eps) {
    __shared__ float part[MF_WAVES];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < MF_WAVES; w++) tot = tot + part[w];
    return 1.0f / sqrtf(tot / (float)k + eps);
}

// Activation source of a fused norm: one f32 residual row x[k] (k <= MF_SEG, a
// multiple of 8) and the norm's f32 weights; stage() writes
// h = f16((x - 0) * r * w + 0), norm_row's expression (nn.rs:142), with r from
// the whole row.
struct SrcNormRow {
    static constexpr int SEG_D = MF_SEG;
    struct Regs {
        float4 x0, x1, w0, w1;
    };
    rsrc_t xr, wr;
    uint32_t k;
    float eps;
    __device__ SrcNormRow(const float *x, const float *w, uint32_t k_, float eps_)
        : xr(make_rsrc(x, k_ * 4u)), wr(make_rsrc(w, k_ * 4u)), k(k_), eps(eps_) {}
    __device__ void load(Regs &a, uint32_t d0, int t) const {
        const uint32_t off = (d0 + 8u * (uint32_t)t) * 4u;  // past k: zeros
        a.x0 = bload16f(xr, off);
        a.x1 = bload16f(xr, off + 16);
        a.w0 = bload16f(wr, off);
        a.w1 = bload16f(wr, off + 16);
    }
    __device__ void stage(uint16_t *a_lds, const Regs &a, int t) const {
        const float xs[8] = {a.x0.x, a.x0.y, a.x0.z, a.x0.w, a.x1.x, a.x1.y, a.x1.z, a.x1.w};
        const float ws[8] = {a.w0.x, a.w0.y, a.w0.z, a.w0.w, a.w1.x, a.w1.y, a.w1.z, a.w1.w};
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) ss = ss + xs[i] * xs[i];
        const float r = rms_scale(ss, k, eps);
        uint16_t h[8];
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = f32_to_f16((xs[i] - 0.0f) * r * ws[i] + 0.0f);
        *(uint4 *)(a_lds + 8 * t) = make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                                               h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
    }
};

// Loads a single-row tile store reads (the residual it adds to, the RoPE
// angles), issued ahead of the next item's weight loads so the store does not
// wait for those.
struct BlkPre {
    float y, c, s;
};
// t: the thread's lane within the tile's store (threadIdx.x when a workgroup
// stores one tile at a time).
template <int STORE>
__device__ __forceinline__ BlkPre blk_prefetch(const Q4GemvArgs &g, const BlkArgs &a, uint32_t tile,
                                               uint32_t t = threadIdx.x) {
    BlkPre p{0.0f, 1.0f, 0.0f};
    if constexpr (STORE == BS_RESID) {
        const uint32_t j = tile * 16 + t;
        if (t < 16 && j < g.n) p.y = a.x[j];
    } else if constexpr (STORE == BS_QKV) {
        const uint32_t pc = tile * 16 + t;
        if (t < 16 && a.cs && pc < (a.heads + a.kv_heads) * a.hd) {
            const uint32_t pi = 8 * ((pc % a.hd) / 16) + (t & 7);
            p.c = a.cs[pi];
            p.s = a.sn[pi];
        }
    }
    return p;
}

// The tile's store from the reduced partials in red (after q4_mfma_reduce).
// pre: blk_prefetch's loads for MR = 1 (MR > 1 reads the residual here).
template <int MR, int STORE>
__device__ __forceinline__ void blk_store(const Q4GemvArgs &g, const BlkArgs &a, uint32_t tile, const float *red,
                                          const BlkPre &pre, int t = (int)threadIdx.x) {
    if constexpr (STORE == BS_RESID) {
        // y += f32(f16(x @ W)): Linear::accumulate's add_f16 (src/convert.rs:37-49)
        if (t < 16 * MR) {
            const int cc = t / MR, r = t % MR;
            const uint32_t j = tile * 16 + cc;
            if (r < (int)g.m && j < g.n) {
                float *yp = a.x + (size_t)r * g.n + j;
                const float y0 = MR == 1 ? pre.y : *yp;
                *yp = y0 + f16_to_f32(f32_to_f16(tile_total<MR>(red, cc, r)));
            }
        }
    } else if constexpr (STORE == BS_GLU) {
        // device tile = 8 gate columns then the same 8 up columns
        if (t < 8 * MR) {
            const int cc = t / MR, r = t % MR;
            const uint32_t jh = tile * 8 + cc;
            if (r < (int)g.m && jh < a.nh) {
                const float gv = f16_to_f32(f32_to_f16(tile_total<MR>(red, cc, r)));
                const float uv = f16_to_f32(f32_to_f16(tile_total<MR>(red, cc + 8, r)));
                a.y[(size_t)r * a.nh + jh] = f32_to_f16(glu_act(a.act, gv) * uv);
            }
        }
    } else {
        static_assert(MR == 1, "the rope / cache store serves one row");
        // device tile = columns 8q..8q+7 and half+8q..half+8q+7 of one head
        // (q heads, then k heads, then v heads): each lane's RoPE partner is
        // lane ^ 8 of the same tile.
        const uint32_t p = tile * 16 + t;
        const uint32_t nq = (a.heads + 2 * a.kv_heads) * a.hd;
        if (t < 16 && p < nq) {
            const uint32_t hd = a.hd, half = hd / 2;
            const uint32_t H = p / hd, qt = (p % hd) / 16, cc = (uint32_t)t;
            const uint32_t i = cc < 8 ? 8 * qt + cc : half + 8 * qt + cc - 8;
            const uint16_t own16 = f32_to_f16(tile_total<1>(red, t, 0));
            const uint16_t par16 = f32_to_f16(tile_total<1>(red, t ^ 8, 0));
            if (H < a.heads + a.kv_heads) {
                float val = f16_to_f32(own16);
                if (a.cs) {
                    const float x1 = f16_to_f32(cc < 8 ? own16 : par16);
                    const float x2 = f16_to_f32(cc < 8 ? par16 : own16);
                    val = cc < 8 ? x1 * pre.c - x2 * pre.s : x2 * pre.c + x1 * pre.s;
                }
                if (H < a.heads) a.q_out[H * hd + i] = f32_to_f16(val * a.scale);
                else a.k_row[(H - a.heads) * hd + i] = f32_to_f16(val);
            } else {
                a.v_row[(H - a.heads - a.kv_heads) * hd + i] = own16;
            }
        }
    }
}

template <int MR, bool NORM, int STORE>
__global__ void __launch_bounds__(MF_WAVES * 64) blk_gemv(Q4GemvArgs g, BlkArgs a) {
    static_assert(!NORM || MR == 1, "the fused norm serves one row");
    static_assert(STORE != BS_QKV || MR == 1, "the rope / cache store serves one row");
    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t *a_lds = (uint16_t *)smem;
    float *red = (float *)smem;
    const uint32_t tile = xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t col = tile * 16 + (threadIdx.x & 15);
    bool timed_out = false;
    float4_t acc;
    if constexpr (NORM) {
        const SrcNormRow src(a.nx, a.nw, g.k, a.eps);
        acc = q4_mfma_mainloop<1, false, SrcNormRow, false>(g, src, ChainArgs{}, a_lds, col, timed_out);
    } else {
        const SrcRows<MR> src(g.lhs, g.m, g.k);
        acc = q4_mfma_mainloop<MR, false, SrcRows<MR>, false>(g, src, ChainArgs{}, a_lds, col, timed_out);
    }
    BlkPre pre{0.0f, 1.0f, 0.0f};
    if constexpr (MR == 1) pre = blk_prefetch<STORE>(g, a, tile);
    q4_mfma_reduce<MR>(acc, red);
    blk_store<MR, STORE>(g, a, tile, red, pre);
}

// The single-row GEMV as a persistent grid (at most BP_WG_PER_CU workgroups a
// CU): each workgroup stages the activation row once -- normalizing it once,
// with the fused norm -- for the whole K (up to BP_MAX_SEG segments), then
// walks its tiles (blockIdx.x, + gridDim.x, ...) segment by segment with
// the next item's weights loading while the current one's MFMAs run.
constexpr int BP_WG_PER_CU = 2;
constexpr int BP_MAX_SEG = 4;  // K <= 16384
constexpr size_t BP_RED_BYTES = MF_WAVES * 16 * 4;
template <bool NORM, int STORE>
__global__ void __launch_bounds__(MF_WAVES * 64) blk_gemv_p(Q4GemvArgs g, BlkArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, c = t & 15;
    const uint32_t ntiles = g.n_pad / 16;
    const uint32_t nseg = (g.nchunks + MF_SEG_CH - 1) / MF_SEG_CH;
    // LDS: red, then the row (whole segments)
    float *red = (float *)smem;
    uint16_t *arow = (uint16_t *)(smem + BP_RED_BYTES);
    const uint32_t mag_lo = __builtin_amdgcn_readfirstlane(0x64006400u) | (uint32_t)(t >> 30);
    const uint32_t mag_hi = __builtin_amdgcn_readfirstlane(0x54005400u) | (uint32_t)(t >> 30);
    const uint32_t mine = (ntiles - 1 - blockIdx.x) / gridDim.x + 1;  // the grid is at most ntiles
    const uint32_t nitems = mine * nseg;
    // item q: tile blockIdx.x + (q / nseg) gridDim.x, segment q % nseg
    auto tile_of = [&](uint32_t q) { return blockIdx.x + (q / nseg) * gridDim.x; };
    auto sc0_of = [&](uint32_t q) { return (q % nseg) * (uint32_t)MF_SEG_CH; };
    Q4Item w0, w1;
    // the activation row first (its loads retire before the weights'), then
    // item 0's weights, then the row staged while those stream in
    if constexpr (NORM) {
        const SrcNormRow src(a.nx, a.nw, g.k, a.eps);
        SrcNormRow::Regs ar;
        src.load(ar, 0, t);
        q4_item_load(g, sc0_of(0), tile_of(0) * 16 + c, w0);
        src.stage(arow, ar, t);
    } else {
        const SrcRows<1> src(g.lhs, 1, g.k);
        SrcRows<1>::Regs ar[BP_MAX_SEG];
#pragma unroll
        for (int sg = 0; sg < BP_MAX_SEG; sg++)
            if ((uint32_t)sg < nseg) src.load(ar[sg], sg * MF_SEG, t);
        q4_item_load(g, sc0_of(0), tile_of(0) * 16 + c, w0);
#pragma unroll
        for (int sg = 0; sg < BP_MAX_SEG; sg++)
            if ((uint32_t)sg < nseg) src.stage(arow + sg * MF_SEG, ar[sg], t);
    }
    __syncthreads();
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t q = 0; q < nitems; q += 2) {
        // clamped past the end: a repeat of the last item (a cache hit), unused
        const uint32_t q1 = q + 1 < nitems ? q + 1 : nitems - 1;
        const uint32_t tq = tile_of(q);
        const bool end0 = q % nseg == nseg - 1;
        BlkPre pre{0.0f, 1.0f, 0.0f};
        if (end0) pre = blk_prefetch<STORE>(g, a, tq);
        q4_item_load(g, sc0_of(q1), tile_of(q1) * 16 + c, w1);
        q4_item_mma1(sc0_of(q), w0, arow, acc, mag_lo, mag_hi);
        if (end0) {
            q4_mfma_reduce<1>(acc, red);
            blk_store<1, STORE>(g, a, tq, red, pre);
            acc = float4_t{0.f, 0.f, 0.f, 0.f};
        }
        if (q + 1 >= nitems) break;
        const uint32_t q2 = q + 2 < nitems ? q + 2 : nitems - 1;
        const uint32_t t1 = tile_of(q1);
        const bool end1 = q1 % nseg == nseg - 1;
        BlkPre pre1{0.0f, 1.0f, 0.0f};
        if (end1) pre1 = blk_prefetch<STORE>(g, a, t1);
        q4_item_load(g, sc0_of(q2), tile_of(q2) * 16 + c, w0);
        q4_item_mma1(sc0_of(q1), w1, arow, acc, mag_lo, mag_hi);
        if (end1) {
            q4_mfma_reduce<1>(acc, red);
            blk_store<1, STORE>(g, a, t1, red, pre1);
            acc = float4_t{0.f, 0.f, 0.f, 0.f};
        }
    }
}


// The single-row GEMV with every weight step in flight (K <= 1024 NS, at most
// TPW tiles a workgroup, one workgroup a compute unit): the weights of all
// its tiles are issued at the start, behind the activation runs, and each
// wave stages only the activations its own chunks multiply (wave w's step u
// multiplies chunks s*128 + 4(w + 8(u%4)) + grp of segment s = u/4), so
// nothing but the fused norm's sum of squares and the partial-tile reduction
// waits on other waves. Two workgroups on one compute unit were measured to
// serialize (the second one's loads queue behind the first one's weights),
// and segment-by-segment loops wait on one segment's weights before the
// next is issued; this form does neither. Step u of a tile reads chunk kc of
// the blocked grid at a constant offset from the wave's first cell; a step
// past K reads zeros (or the grid's padding, with its scale replaced by 0).
template <bool NORM, int STORE, int TPW, int NS>
__global__ void __launch_bounds__(MF_WAVES * 64) blk_gemv_w(Q4GemvArgs g, BlkArgs a) {
    constexpr int NSEG = (NS + 3) / 4;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, c = lane & 15, grp = lane >> 4;
    uint16_t *wlds = (uint16_t *)smem + wave * (NSEG * 512);  // this wave's runs [NSEG][4][128]
    float *red = (float *)(smem + MF_WAVES * NSEG * 1024);    // [TPW][MF_WAVES][16]
    const uint32_t ntiles = g.n_pad / 16, G = gridDim.x;
    const uint32_t mag_lo = __builtin_amdgcn_readfirstlane(0x64006400u) | (uint32_t)(t >> 30);
    const uint32_t mag_hi = __builtin_amdgcn_readfirstlane(0x54005400u) | (uint32_t)(t >> 30);

    // -- 1. the wave's activation runs (lane (grp, c): 8 depths of run grp of
    //       each segment), then every tile's weight steps
    uint4 ah[NSEG];
    float4 ax[NSEG][2], aw[NSEG][2];
#pragma unroll
    for (int sg = 0; sg < NSEG; sg++) {
        const uint32_t da = (sg * 128u + 4u * (wave + MF_WAVES * grp)) * Q4_CHUNK + (uint32_t)c * 8u;
        if constexpr (NORM) {
            const rsrc_t xr = make_rsrc(a.nx, g.k * 4u), wr = make_rsrc(a.nw, g.k * 4u);
            const uint32_t off = da < g.k ? da * 4u : OOB;
            ax[sg][0] = bload16f(xr, off);
            ax[sg][1] = bload16f(xr, da < g.k ? off + 16 : OOB);
            aw[sg][0] = bload16f(wr, off);
            aw[sg][1] = bload16f(wr, da < g.k ? off + 16 : OOB);
        } else {
            ah[sg] = bload16(make_rsrc(g.lhs, g.k * 2u), da < g.k ? da * 2u : OOB);
        }
    }
    const uint32_t grid_rows = (g.nchunks + 3) & ~3u;
    const rsrc_t nr = make_rsrc(g.nib, grid_rows * g.n_pad * 16u), sr = make_rsrc(g.sc, grid_rows * g.n_pad * 2u);
    bool live[TPW];
    uint32_t tile[TPW];
    uint4 wq[TPW][NS];
    uint16_t sv[TPW][NS];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const uint32_t li = blockIdx.x + j * G;
        live[j] = li < ntiles;
        tile[j] = xcd_tile(live[j] ? li : 0, ntiles);
        const uint32_t col = tile[j] * 16 + c;
        const uint32_t cell0 = wave * 4u * g.n_pad + grp * 16u + (col >> 4) * 64u + (col & 15);
#pragma unroll
        for (int u = 0; u < NS; u++) {
            const uint32_t kc = (u / 4) * 128u + 4u * (wave + MF_WAVES * (u % 4)) + grp;
            const uint32_t cell = cell0 + ((u / 4) * 32u + MF_WAVES * (u % 4)) * 4u * g.n_pad;
            wq[j][u] = bload16_nt(nr, live[j] ? cell * 16u : OOB);
            const uint16_t sl = bload2_nt(sr, live[j] ? cell * 2u : OOB);
            sv[j][u] = kc < g.nchunks ? sl : (uint16_t)0;
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // the stores' own loads (threads 16 j .. 16 j + 15 store tile j)
    const int sj = t >> 4, st = t & 15;
    BlkPre pre{0.0f, 1.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < TPW; j++)
        if (sj == j && live[j]) pre = blk_prefetch<STORE>(g, a, tile[j], (uint32_t)st);

    // -- 2. stage the wave's runs (with the fused norm: h = f16(x r w), r
    //       from the whole row's sum of squares, nn.rs:127-144)
    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int sg = 0; sg < NSEG; sg++) {
            const float xs[8] = {ax[sg][0].x, ax[sg][0].y, ax[sg][0].z, ax[sg][0].w,
                                 ax[sg][1].x, ax[sg][1].y, ax[sg][1].z, ax[sg][1].w};
#pragma unroll
            for (int i = 0; i < 8; i++) ss = ss + xs[i] * xs[i];
        }
        const float r = rms_scale(ss, g.k, a.eps);
#pragma unroll
        for (int sg = 0; sg < NSEG; sg++) {
            const float xs[8] = {ax[sg][0].x, ax[sg][0].y, ax[sg][0].z, ax[sg][0].w,
                                 ax[sg][1].x, ax[sg][1].y, ax[sg][1].z, ax[sg][1].w};
            const float ws[8] = {aw[sg][0].x, aw[sg][0].y, aw[sg][0].z, aw[sg][0].w,
                                 aw[sg][1].x, aw[sg][1].y, aw[sg][1].z, aw[sg][1].w};
            uint16_t h[8];
#pragma unroll
            for (int i = 0; i < 8; i++) h[i] = f32_to_f16((xs[i] - 0.0f) * r * ws[i] + 0.0f);
            *(uint4 *)(wlds + sg * 512 + lane * 8) =
                make_uint4(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                           h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16));
        }
    } else {
#pragma unroll
        for (int sg = 0; sg < NSEG; sg++) *(uint4 *)(wlds + sg * 512 + lane * 8) = ah[sg];
    }

    // -- 3. dequant + MFMA, step by step as the weights land (every B lane
    //       reads row 0: only output row 0 is used)
    float4_t acc[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        acc[j] = (float4_t){0.f, 0.f, 0.f, 0.f};
        if (!live[j]) continue;  // uniform
#pragma unroll
        for (int u = 0; u < NS; u++) {
            uint4 ab[4];
#pragma unroll
            for (int w = 0; w < 4; w++) ab[w] = *(const uint4 *)(wlds + (u / 4) * 512 + (u % 4) * 128 + grp * 32 + w * 8);
            const half2_t s2 = {__builtin_bit_cast(_Float16, sv[j][u]), __builtin_bit_cast(_Float16, sv[j][u])};
            const uint32_t words[4] = {wq[j][u].x, wq[j][u].y, wq[j][u].z, wq[j][u].w};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint4 wa = q4_deq8(words[w], s2, mag_lo, mag_hi);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, wa),
                                                                __builtin_bit_cast(half8_t, ab[w]), acc[j], 0, 0, 0);
            }
        }
    }
    // -- 4. the waves' partial tiles in fixed order, then each tile's store
    if (c == 0) {
#pragma unroll
        for (int j = 0; j < TPW; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) red[(j * MF_WAVES + wave) * 16 + 4 * grp + v] = acc[j][v];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPW; j++)
        if (sj == j && live[j]) blk_store<1, STORE>(g, a, tile[j], red + j * MF_WAVES * 16, pre, st);
}

template <bool NORM, int STORE, int TPW, int NS>
hipError_t launch_blk_w(const Q4GemvArgs &g, const BlkArgs &a, uint32_t grid, hipStream_t s) {
    constexpr size_t lds = (size_t)MF_WAVES * ((NS + 3) / 4) * 1024 + (size_t)TPW * MF_WAVES * 16 * 4;
    hipLaunchKernelGGL((blk_gemv_w<NORM, STORE, TPW, NS>), dim3(grid), dim3(MF_WAVES * 64), lds, s, g, a);
    return hipGetLastError();
}

// blk_gemv_w when it serves the call (one row, block 32, K within 16 steps a
// lane -- 4 with the fused norm or two tiles a compute unit -- and at most
// two tiles a compute unit): the qkv, out and down projections. Wider
// projections (the 28672-column gate/up) keep blk_gemv_p's two-workgroup
// ring: all seven tiles of a compute unit in flight at once measured 20.7
// against 16.3 us there. hipErrorNotSupported otherwise.
template <bool NORM, int STORE>
hipError_t try_blk_w(const Q4GemvArgs &g, const BlkArgs &a, size_t m, hipStream_t s) {
    const uint32_t ntiles = g.n_pad / 16;
    const uint32_t grid = std::min<uint32_t>(ntiles, (uint32_t)device_cus());
    const uint32_t tpw = grid ? (ntiles + grid - 1) / grid : 0;
    const uint32_t ns = (g.nchunks + 31) / 32;  // steps a lane: 32 chunks a step across the workgroup
    if (m != 1 || g.block_shift != 5 || (g.k & 7) != 0 || grid == 0 || tpw > 2 || ns > 16 ||
        cell_grid_rows(g.nchunks) * (size_t)g.n_pad * 16 >= ((size_t)1 << 31) || ((NORM || tpw > 1) && ns > 4))
        return hipErrorNotSupported;
    if (tpw == 2) return launch_blk_w<NORM, STORE, 2, 4>(g, a, grid, s);
    if (ns <= 4) return launch_blk_w<NORM, STORE, 1, 4>(g, a, grid, s);
    if constexpr (NORM) {
        return hipErrorNotSupported;
    } else {
        if (ns <= 8) return launch_blk_w<NORM, STORE, 1, 8>(g, a, grid, s);
        if (ns <= 14) return launch_blk_w<NORM, STORE, 1, 14>(g, a, grid, s);
        return launch_blk_w<NORM, STORE, 1, 16>(g, a, grid, s);
    }
}

template <int MR, bool NORM, int STORE>
hipError_t launch_blk(const Q4GemvArgs &g, const BlkArgs &a, hipStream_t s) {
    hipLaunchKernelGGL((blk_gemv<MR, NORM, STORE>), dim3(g.n_pad / 16), dim3(MF_WAVES * 64),
                       q4_mfma_lds_bytes<MR>(), s, g, a);
    return hipGetLastError();
}

template <bool NORM, int STORE>
hipError_t launch_blk_p(const Q4GemvArgs &g, const BlkArgs &a, hipStream_t s) {
    const uint32_t ntiles = g.n_pad / 16;
    const uint32_t nseg = (g.nchunks + MF_SEG_CH - 1) / MF_SEG_CH;
    const uint32_t grid = std::min<uint32_t>(ntiles, (uint32_t)(BP_WG_PER_CU * device_cus()));
    const size_t lds = BP_RED_BYTES + (size_t)nseg * MF_SEG * 2;
    hipLaunchKernelGGL((blk_gemv_p<NORM, STORE>), dim3(grid), dim3(MF_WAVES * 64), lds, s, g, a);
    return hipGetLastError();
}

// One row with at least two tiles for every workgroup of a full persistent
// grid (K within its staging): the persistent grid, which then keeps the
// next tile's weights in flight and normalizes the row once per workgroup
// rather than once per tile. Fewer tiles (a workgroup would get about one)
// run faster as one workgroup per tile (measured on the block's projections:
// 28672 columns 15.7 vs 18.4 us, 4096-6144 columns 0.3-0.4 us slower).
template <bool NORM, int STORE>
hipError_t launch_blk_rows(const Q4GemvArgs &g, const BlkArgs &a, size_t m, hipStream_t s) {
    {
        const hipError_t e = try_blk_w<NORM, STORE>(g, a, m, s);
        if (e != hipErrorNotSupported) return e;
    }
    const bool persistent = m == 1 && (g.nchunks + MF_SEG_CH - 1) / MF_SEG_CH <= (uint32_t)BP_MAX_SEG &&
                            g.n_pad / 16 >= 2u * BP_WG_PER_CU * (uint32_t)device_cus();
    if constexpr (NORM || STORE == BS_QKV) {
        if (m != 1) return hipErrorNotSupported;
        if (persistent) return launch_blk_p<NORM, STORE>(g, a, s);
        return launch_blk<1, NORM, STORE>(g, a, s);
    } else {
        if (persistent) return launch_blk_p<NORM, STORE>(g, a, s);
        if (m <= 1) return launch_blk<1, NORM, STORE>(g, a, s);
        if (m <= 2) return launch_blk<2, NORM, STORE>(g, a, s);
        if (m <= 4) return launch_blk<4, NORM, STORE>(g, a, s);
        return launch_blk<8, NORM, STORE>(g, a, s);
    }
}

// ---------------------------------------------------------------------------
// Attention over the f16 cache (one query row)
// ---------------------------------------------------------------------------
constexpr int AT_T = 256;    // threads
constexpr int AT_KPS = 64;   // keys per split (one per lane of the softmax wave)
constexpr int AT_HC = 4;     // query heads per workgroup (a chunk of one KV head's group)


// LPK lanes per key (8 depths each: head_dim <= 8 * LPK). Thread t takes key
// slot t / LPK of each 256/LPK-key step and depths 8 (t % LPK) .. +8; all
// its key, value and query loads are issued before the first is used.
template <int LPK>
__global__ void __launch_bounds__(AT_T) attn_split(AttnArgs a) {
    constexpr int KPI = AT_T / LPK;   // keys per step
    constexpr int IT = AT_KPS / KPI;  // steps per split
    constexpr int HDM = 8 * LPK;      // largest head_dim served
    __shared__ float sc[AT_HC][AT_KPS];
    __shared__ float ored[KPI][AT_HC][HDM];
    __shared__ float2 mls[AT_HC];
    const int t = threadIdx.x;
    const int ks = t / LPK, c = t % LPK;
    const uint32_t split = blockIdx.x, row = blockIdx.z;
    const uint32_t len = a.len + row;  // this row's causal prefix
    if (split * AT_KPS >= len) return;  // past the row's last split (uniform: before any barrier)
    const uint32_t kvh = blockIdx.y / a.hchunks, hc0 = (blockIdx.y % a.hchunks) * AT_HC;
    const bool dim_ok = 8u * c < a.hd;
    const rsrc_t qr = make_rsrc(a.q + (size_t)row * a.heads * a.hd, a.heads * a.hd * 2u);
    const rsrc_t kr = make_rsrc(a.k, len * a.ld * 2u);
    const rsrc_t vr = make_rsrc(a.v, len * a.ld * 2u);
    float *po = a.po + (size_t)row * a.nsplit * a.heads * a.hd;
    float2 *pml = a.pml + (size_t)row * a.nsplit * a.heads;
    uint4 qv[AT_HC];
#pragma unroll
    for (int hh = 0; hh < AT_HC; hh++) {
        const uint32_t h = kvh * a.group + hc0 + hh;
        const bool ok = dim_ok && hc0 + hh < a.group;
        qv[hh] = bload16(qr, ok ? (h * a.hd + 8 * c) * 2u : OOB);
    }
    const uint32_t key0 = split * AT_KPS;
    uint4 kv[IT], vv[IT];
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const uint32_t key = key0 + ks + KPI * it;
        const uint32_t off = (key < len && dim_ok) ? (key * a.ld + kvh * a.hd + 8 * c) * 2u : OOB;
        kv[it] = bload16(kr, off);
        vv[it] = bload16(vr, off);
    }
    // scores: q . k over this lane's 8 depths, summed over the key's lanes
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const uint32_t key = key0 + ks + KPI * it;
        const uint32_t kw[4] = {kv[it].x, kv[it].y, kv[it].z, kv[it].w};
#pragma unroll
        for (int hh = 0; hh < AT_HC; hh++) {
            const uint32_t qw[4] = {qv[hh].x, qv[hh].y, qv[hh].z, qv[hh].w};
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++)
                s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, qw[w]), __builtin_bit_cast(half2_t, kw[w]),
                                           s, false);
            s = dpp_group_sum<LPK>(s);
            if (c == 0) sc[hh][ks + KPI * it] = key < len ? s : -INFINITY;
        }
    }
    __syncthreads();
    // softmax within the split: wave w takes query head w of the chunk
    {
        const int wave = t >> 6, lane = t & 63;
        for (int hh = wave; hh < AT_HC; hh += AT_T / 64) {
            const float v = sc[hh][lane];
            const float m = wave_max(v);
            const float p = v == -INFINITY ? 0.0f : expf(v - m);
            const float l = wave_sum(p);
            sc[hh][lane] = p;
            if (lane == 0) mls[hh] = make_float2(m, l);
        }
    }
    __syncthreads();
    // value sums: this lane's 8 depths over its keys, then over the key slots
    float acc[AT_HC][8];
#pragma unroll
    for (int hh = 0; hh < AT_HC; hh++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[hh][e] = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const uint32_t vw[4] = {vv[it].x, vv[it].y, vv[it].z, vv[it].w};
        float vf[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            vf[2 * w] = f16_to_f32((uint16_t)vw[w]);
            vf[2 * w + 1] = f16_to_f32((uint16_t)(vw[w] >> 16));
        }
#pragma unroll
        for (int hh = 0; hh < AT_HC; hh++) {
            const float p = sc[hh][ks + KPI * it];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[hh][e] = __builtin_fmaf(p, vf[e], acc[hh][e]);
        }
    }
#pragma unroll
    for (int hh = 0; hh < AT_HC; hh++)
#pragma unroll
        for (int e = 0; e < 8; e++) ored[ks][hh][8 * c + e] = acc[hh][e];
    __syncthreads();
    for (int o = t; o < AT_HC * HDM; o += AT_T) {
        const uint32_t hh = (uint32_t)o / HDM, d = (uint32_t)o % HDM;
        if (d < a.hd && hc0 + hh < a.group) {
            float sum = 0.0f;
            for (int q = 0; q < KPI; q++) sum = sum + ored[q][hh][d];
            const uint32_t h = kvh * a.group + hc0 + hh;
            po[((size_t)split * a.heads + h) * a.hd + d] = sum;
        }
    }
    if (t < AT_HC && hc0 + t < a.group) pml[(size_t)split * a.heads + kvh * a.group + hc0 + t] = mls[t];
}

// The splits of head blockIdx.x merged, for depths 16 blockIdx.y .. +16:
// o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, f16 (the out
// projection's input) or f32. Thread (group g = t / 16, depth t % 16) takes
// splits g, g + 16, ...: it issues the loads of CM_P of them at once, then
// folds them into its running (m, l, o) -- rescaled by e^(m_old - m_new) --
// so a context of up to 16 CM_P splits costs one memory round trip; the 16
// groups' (m, l, o) are then merged through LDS in group order.
constexpr int CM_T = 256;           // threads
constexpr int CM_D = 16;            // depths per workgroup
constexpr int CM_G = CM_T / CM_D;   // split groups
constexpr int CM_P = 8;             // splits per thread per round trip
// Row blockIdx.z merges its own splits: attn_splits(len0 + row) of the
// nsplit_max allotted to each row.
template <bool F16OUT>
__global__ void __launch_bounds__(CM_T) attn_combine(const float *po, const float2 *pml, uint32_t nsplit_max,
                                                     uint32_t len0, uint32_t heads, uint32_t hd, void *out) {
    __shared__ float sm[CM_G][CM_D], sl[CM_G][CM_D], so[CM_G][CM_D];
    const uint32_t h = blockIdx.x, t = threadIdx.x, row = blockIdx.z;
    const uint32_t nsplit = (len0 + row + AT_KPS - 1) / AT_KPS;
    po += (size_t)row * nsplit_max * heads * hd;
    pml += (size_t)row * nsplit_max * heads;
    out = F16OUT ? (void *)((uint16_t *)out + (size_t)row * heads * hd) : (void *)((float *)out + (size_t)row * heads * hd);
    const uint32_t dl = t % CM_D, g = t / CM_D;
    const uint32_t d = blockIdx.y * CM_D + dl;
    const bool dok = d < hd;
    float m = -INFINITY, l = 0.0f, o = 0.0f;
    for (uint32_t s0 = g; s0 < nsplit; s0 += CM_G * CM_P) {
        float2 ml[CM_P];
        float ov[CM_P];
#pragma unroll
        for (int j = 0; j < CM_P; j++) {
            const uint32_t s = s0 + CM_G * j;
            const bool ok = s < nsplit;
            ml[j] = ok ? pml[(size_t)s * heads + h] : make_float2(-INFINITY, 0.0f);
            ov[j] = ok && dok ? po[((size_t)s * heads + h) * hd + d] : 0.0f;
        }
        // split s0 exists, and every split holds at least one key: mc is finite
        float mc = m;
#pragma unroll
        for (int j = 0; j < CM_P; j++) mc = fmaxf(mc, ml[j].x);
        const float r = expf(m - mc);
        l = l * r;
        o = o * r;
#pragma unroll
        for (int j = 0; j < CM_P; j++) {
            const float w = expf(ml[j].x - mc);
            l = __builtin_fmaf(w, ml[j].y, l);
            o = __builtin_fmaf(w, ov[j], o);
        }
        m = mc;
    }
    sm[g][dl] = m;
    sl[g][dl] = l;
    so[g][dl] = o;
    __syncthreads();
    if (t < CM_D && dok) {
        float mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < CM_G; q++) mx = fmaxf(mx, sm[q][t]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int q = 0; q < CM_G; q++) {
            const float w = expf(sm[q][t] - mx);  // a group with no split: e^-inf = 0
            lt = __builtin_fmaf(w, sl[q][t], lt);
            ot = __builtin_fmaf(w, so[q][t], ot);
        }
        const float v = ot / lt;
        if (F16OUT) ((uint16_t *)out)[h * hd + d] = f32_to_f16(v);
        else ((float *)out)[h * hd + d] = v;
    }
}

// ---------------------------------------------------------------------------
// Causal attention of a block of query rows on the matrix cores
// ---------------------------------------------------------------------------
// For blocks of at least AP_MIN_ROWS rows (attention_kv_causal_f16's blocked
// path, src/kernels/kv_attention.rs:198-201 with csrc/attention_kv_sme.h: the
// same arithmetic as the one-row call -- q * scale rounded to f16, f32 scores
// from f16 products, f32 exp, probabilities rounded to f16, f32 sums of p * v
// -- with both products on the matrix unit, so only the order of the sums
// differs; the reference holds such rows to 1e-3 of the one-row call). A
// workgroup takes one KV head, a chunk of up to 4 of its query heads (one a
// wave) and AP_BR consecutive query positions, and walks the keys of its last
// position in blocks of AP_KB: the block's keys and values go global ->
// registers (the next block's while this one is multiplied) -> LDS, keys
// row-major and values transposed; each wave then forms S^T = K Q^T for its
// head (v_mfma_f32_16x16x32_f16: A = 16 keys x 32 depths read from LDS, B =
// its 16 query rows, kept in registers), masks keys past each row's own
// position, updates the rows' running max and sum (flash attention's
// rescale), and adds O^T += V^T P^T (v_mfma_f32_16x16x16_f16: A = 16 depths x
// 4 keys of the transposed values, B = the f16 probabilities, which S^T's
// accumulator layout already holds as that operand: lane l has row l % 16 and
// keys 4 (l / 16) .. + 3 of a 16-key tile). Every lane's accumulators belong to
// its row l % 16, so the rescale and the final o / l need no exchange.
constexpr int AP_T = 256, AP_KB = 64, AP_BR = 16;
constexpr uint32_t AP_MIN_ROWS = 32;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float xor_lanes(float v, int m) { return __shfl_xor(v, m, 64); }

template <int HDM>
__global__ void __launch_bounds__(AP_T) attn_rows_mfma(AttnArgs a) {
    constexpr int KK = HDM / 32;  // 32-depth steps of the scores
    constexpr int DT = HDM / 16;  // 16-depth tiles of the output
    constexpr int LJ = HDM / 32;  // 16-byte loads a thread a block, of keys and of values
    constexpr int KS = HDM + 8;   // key row stride in LDS (halfs)
    constexpr int VS = AP_KB + 4; // transposed value row stride (halfs): conflict-free 8-byte reads
    __shared__ __align__(16) uint16_t k_lds[AP_KB * KS];
    __shared__ __align__(16) uint16_t v_lds[HDM * VS];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, r16 = lane & 15, g4 = lane >> 4;
    // unit u: head chunk u % ny, position tile u / ny (consecutive units, which
    // the dispatcher spreads over the XCDs, take one tile's head chunks, so the
    // workgroups of one KV head share an XCD's L2 when ny is a multiple of 8)
    const uint32_t ny = (a.heads / a.group) * a.hchunks, yc = blockIdx.x % ny;
    const uint32_t p0 = (blockIdx.x / ny) * AP_BR;
    const uint32_t kvh = yc / a.hchunks, hc0 = (yc % a.hchunks) * AT_HC;
    const bool head_ok = hc0 + wave < a.group;  // uniform per wave
    const uint32_t h = kvh * a.group + hc0 + wave;
    const uint32_t pend = min(p0 + AP_BR, a.rows);
    const uint32_t nkeys = a.len + pend - 1;  // the last position's prefix
    const uint32_t nblk = (nkeys + AP_KB - 1) / AP_KB;
    const uint32_t row = p0 + r16;  // this lane's query position (of the block)
    const bool rok = head_ok && row < a.rows;
    const uint32_t lim = a.len + row;  // its keys: 0 .. lim - 1

    // the wave's 16 query rows of head h (B operand of the scores)
    const rsrc_t qr = make_rsrc(a.q, a.rows * a.heads * a.hd * 2u);
    uint4 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        const uint32_t d = 32u * kk + 8u * g4;
        qf[kk] = bload16(qr, rok && d < a.hd ? ((row * a.heads + h) * a.hd + d) * 2u : OOB);
    }
    // a block's keys and values: thread t loads key t % 64, depths 8 ((t / 64) + 4 j) .. + 8
    const rsrc_t kr = make_rsrc(a.k, nkeys * a.ld * 2u), vr = make_rsrc(a.v, nkeys * a.ld * 2u);
    // two blocks' keys and values in flight in registers (sets A and B)
    uint4 ka_[LJ], va_[LJ], kb_[LJ], vb_[LJ];
    auto load_blk = [&](uint32_t b, uint4 (&kreg)[LJ], uint4 (&vreg)[LJ]) __attribute__((always_inline)) {
        const uint32_t key = b * AP_KB + (uint32_t)(t & 63);
#pragma unroll
        for (int j = 0; j < LJ; j++) {
            const uint32_t d = (uint32_t)((t >> 6) + 4 * j) * 8u;
            const uint32_t off = b < nblk && key < nkeys && d < a.hd ? (key * a.ld + kvh * a.hd + d) * 2u : OOB;
            kreg[j] = bload16(kr, off);
            vreg[j] = bload16(vr, off);
        }
    };
    auto store_blk = [&](const uint4 (&kreg)[LJ], const uint4 (&vreg)[LJ]) __attribute__((always_inline)) {
        const int key = t & 63;
#pragma unroll
        for (int j = 0; j < LJ; j++) {
            const int d0 = ((t >> 6) + 4 * j) * 8;
            *(uint4 *)(k_lds + key * KS + d0) = kreg[j];
            const uint32_t w[4] = {vreg[j].x, vreg[j].y, vreg[j].z, vreg[j].w};
#pragma unroll
            for (int e = 0; e < 8; e++) v_lds[(d0 + e) * VS + key] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    float4_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = (float4_t){0.f, 0.f, 0.f, 0.f};
    // block b: its registers to LDS, then block b + 2's loads into them (a
    // block past the last loads nothing: every offset out of range)
    auto block = [&](uint32_t b, uint4 (&kreg)[LJ], uint4 (&vreg)[LJ]) __attribute__((always_inline)) {
        __syncthreads();  // the previous block's LDS readers are done
        store_blk(kreg, vreg);
        load_blk(b + 2, kreg, vreg);
        __syncthreads();
        if (!head_ok) return;
        // S^T for the block's 4 key tiles
        float4_t sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            sc[kt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const uint4 ka = *(const uint4 *)(k_lds + (16 * kt + r16) * KS + 32 * kk + 8 * g4);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, ka),
                                                                __builtin_bit_cast(half8_t, qf[kk]), sc[kt], 0, 0, 0);
            }
        }
        // causal mask (only in the blocks that reach past the first row's
        // prefix, or for rows past the block), the block's row max and the
        // running rescale
        float mb = -INFINITY;
        if ((b + 1) * AP_KB > a.len + p0 || pend - p0 < (uint32_t)AP_BR) {
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const uint32_t key = b * AP_KB + 16u * kt + 4u * g4 + v;
                    if (!rok || key >= lim) sc[kt][v] = -INFINITY;
                }
        }
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) mb = fmaxf(mb, sc[kt][v]);
        mb = fmaxf(mb, xor_lanes(mb, 16));
        mb = fmaxf(mb, xor_lanes(mb, 32));
        const float mn = fmaxf(m_run, mb);
        // e^(x - mn) as the hardware 2^(x log2 e - mn log2 e) (v_exp_f32;
        // the blocked form's rounding of p to f16 dominates its error); a row
        // with no key yet keeps p = 0 (2^-inf)
        constexpr float LOG2E = 1.4426950408889634f;
        const float nb2 = mn == -INFINITY ? 0.0f : -mn * LOG2E;
        const float alpha = m_run == mn ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m_run, LOG2E, nb2));
        float ps = 0.0f;
        half4_t pf[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][v], LOG2E, nb2));
                ps = ps + p;
                pf[kt][v] = (_Float16)p;
            }
        ps = ps + xor_lanes(ps, 16);
        ps = ps + xor_lanes(ps, 32);
        l_run = __builtin_fmaf(l_run, alpha, ps);
        m_run = mn;
        // O^T += V^T P^T (the rescale only when some row's max moved)
        const bool moved = __builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            if (moved) o[dt] = o[dt] * alpha;
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                const uint2 va = *(const uint2 *)(v_lds + (16 * dt + r16) * VS + 16 * kt + 4 * g4);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, va), pf[kt], o[dt], 0, 0,
                                                              0);
            }
        }
    };
    load_blk(0, ka_, va_);
    load_blk(1, kb_, vb_);
    for (uint32_t b = 0; b < nblk; b += 2) {
        block(b, ka_, va_);
        if (b + 1 < nblk) block(b + 1, kb_, vb_);
    }
    if (!rok) return;
    const size_t base = ((size_t)row * a.heads + h) * a.hd;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint32_t d = 16u * dt + 4u * g4 + v;
            if (d >= a.hd) continue;
            const float val = o[dt][v] / l_run;
            if (a.f16_out) ((uint16_t *)a.out)[base + d] = f32_to_f16(val);
            else ((float *)a.out)[base + d] = val;
        }
}

// m rows of the qkv projection (an f16 GEMM output in the fused QKV store's
// device column order: a 16-column tile holds depths 8q..8q+7 and
// half+8q..half+8q+7 of one head, each RoPE pair in lanes c, c ^ 8) to the
// attention's inputs at positions pos0 + r, with the fused store's arithmetic
// (the rotation in f32 of the f16 outputs, x1 c - x2 s and x2 c + x1 s as
// examples/bonsai/model.rs:87-99; q16 = f16(q * scale), kv_attention.rs:298-302;
// k rounded to f16, v copied). One thread per (row, column).
__global__ void __launch_bounds__(256) qkv_rows(QkvRowsArgs a) {
    const uint32_t r = blockIdx.y;
    const uint32_t n = (a.heads + 2 * a.kv_heads) * a.hd;
    const uint32_t p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n) return;
    const uint32_t hd = a.hd, half = hd / 2;
    const uint32_t H = p / hd, qt = (p % hd) / 16, cc = p % 16;
    const uint32_t i = cc < 8 ? 8 * qt + cc : half + 8 * qt + cc - 8;
    const uint16_t *row = a.qkv + (size_t)r * n;
    const uint16_t own16 = row[p];
    const size_t ld = (size_t)a.kv_heads * hd;
    if (H < a.heads + a.kv_heads) {
        float val = f16_to_f32(own16);
        if (a.cs) {
            const uint16_t par16 = row[p ^ 8];
            const uint32_t pi = 8 * qt + (cc & 7);
            const float c = a.cs[(size_t)r * half + pi], s = a.sn[(size_t)r * half + pi];
            const float x1 = f16_to_f32(cc < 8 ? own16 : par16);
            const float x2 = f16_to_f32(cc < 8 ? par16 : own16);
            val = cc < 8 ? x1 * c - x2 * s : x2 * c + x1 * s;
        }
        if (H < a.heads) a.q_out[(size_t)r * a.heads * hd + H * hd + i] = f32_to_f16(val * a.scale);
        else a.k_cache[(size_t)r * ld + (H - a.heads) * hd + i] = f32_to_f16(val);
    } else {
        a.v_cache[(size_t)r * ld + (H - a.heads - a.kv_heads) * hd + i] = own16;
    }
}

// The sum of each thread's f32 partial over the workgroup (MF_WAVES waves):
// a wave reduction, then the waves' sums in wave order (every thread gets the
// same bits). part: MF_WAVES floats of LDS, free on entry and on return.
__device__ __forceinline__ float wg_sum(float v, float *part) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < MF_WAVES; w++) tot = tot + part[w];
    __syncthreads();
    return tot;
}

// One row per workgroup of nn::layer_norm (LAYER: mean, then the variance
// about it, two passes in f32; out = (v - mean) * r * w + b, nn.rs:133-143) or
// nn::rms_norm (mean 0, no bias), r = 1 / sqrt(var + eps), into f16. The sums
// run in another order than lane_sum's, so the f16 outputs agree with the
// portable path's within an f16 rounding.
template <bool LAYER>
__global__ void __launch_bounds__(MF_WAVES * 64) norm_rows(const float *x, const float *w, const float *b,
                                                           uint32_t dim, float eps, uint16_t *y) {
    __shared__ float part[MF_WAVES];
    const float *xr = x + (size_t)blockIdx.x * dim;
    float mean = 0.0f;
    if constexpr (LAYER) {
        float s = 0.0f;
        for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) s = s + xr[i];
        mean = wg_sum(s, part) / (float)dim;
    }
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) {
        const float d = xr[i] - mean;
        ss = ss + d * d;
    }
    const float r = 1.0f / sqrtf(wg_sum(ss, part) / (float)dim + eps);
    for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x)
        y[(size_t)blockIdx.x * dim + i] = f32_to_f16((xr[i] - mean) * r * w[i] + (b ? b[i] : 0.0f));
}

// q (f32) to the rounded query attention_kv_f16 scores with: f16(q * scale).
__global__ void attn_round_q(const float *q, float scale, uint32_t count, uint16_t *qh) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) qh[i] = f32_to_f16(q[i] * scale);
}

// ---------------------------------------------------------------------------
// Stand-alone row passes
// ---------------------------------------------------------------------------
// nn::rms_norm into f16, one workgroup of MF_WAVES waves per row.
__global__ void __launch_bounds__(MF_WAVES * 64) rms_norm_rows(const float *x, const float *w, uint32_t dim,
                                                               float eps, uint16_t *y) {
    const float *xr = x + (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) ss = ss + xr[i] * xr[i];
    const float r = rms_scale(ss, dim, eps);
    for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x)
        y[(size_t)blockIdx.x * dim + i] = f32_to_f16((xr[i] - 0.0f) * r * w[i] + 0.0f);
}

// glu over rows of 2n gate / up values: the reference's layout (each
// 32-column chunk, the last w < 32 wide, gate then up: linear.rs:601-619,
// 803-826) or the device tiles of 8 gate + 8 up columns (tile8).
__global__ void glu_rows(const uint16_t *both, uint32_t m, uint32_t n, uint32_t act, int tile8, uint16_t *y) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)m * n) return;
    const uint32_t r = (uint32_t)(idx / n), j = (uint32_t)(idx % n);
    const uint32_t stride = tile8 ? 16 * ((n + 7) / 8) : 2 * n;  // tiles pad to whole 16-column tiles
    const uint16_t *row = both + (size_t)r * stride;
    uint32_t gi, ui;
    if (tile8) {
        gi = 16 * (j / 8) + j % 8;
        ui = gi + 8;
    } else {
        const uint32_t c0 = j / 32 * 32, w = n - c0 < 32 ? n - c0 : 32;
        gi = 2 * c0 + (j - c0);
        ui = gi + w;
    }
    y[idx] = f32_to_f16(glu_act(act, f16_to_f32(row[gi])) * f16_to_f32(row[ui]));
}

__global__ void add_f16_values(const uint16_t *h, uint64_t count, float *y) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) y[i] = y[i] + f16_to_f32(h[i]);
}

}  // namespace

hipError_t launch_blk_gemv(const WDev &w, size_t m, const uint16_t *lhs, const BlkArgs &a, int store,
                           bool norm, hipStream_t s) {
    if (w.kind != W_Q4 || w.mins || w.block < (size_t)Q4_CHUNK || w.nchunks == 0 || m == 0 || m > 8)
        return hipErrorNotSupported;
    if (norm && (w.k > (size_t)MF_SEG || w.k % 8 != 0)) return hipErrorNotSupported;
    if ((size_t)m * w.k * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    const Q4GemvArgs g = q4_gemv_args(w, m, nullptr, lhs);
    switch (store) {
    case BS_RESID:
        return norm ? launch_blk_rows<true, BS_RESID>(g, a, m, s) : launch_blk_rows<false, BS_RESID>(g, a, m, s);
    case BS_GLU:
        return norm ? launch_blk_rows<true, BS_GLU>(g, a, m, s) : launch_blk_rows<false, BS_GLU>(g, a, m, s);
    case BS_QKV:
        return norm ? launch_blk_rows<true, BS_QKV>(g, a, m, s) : launch_blk_rows<false, BS_QKV>(g, a, m, s);
    default:
        return hipErrorInvalidValue;
    }
}

size_t attn_splits(size_t len) { return (len + AT_KPS - 1) / AT_KPS; }

size_t attn_partial_floats(size_t rows, size_t last_len, size_t heads, size_t hd) {
    return std::max<size_t>(rows, 1) * attn_splits(last_len) * heads * (hd + 2);
}

bool attn_rows_blocked(size_t rows) { return rows >= AP_MIN_ROWS; }

hipError_t launch_attention(const AttnArgs &a0, void *out, bool f16_out, hipStream_t s) {
    AttnArgs a = a0;
    if (a.rows == 0) a.rows = 1;
    if (a.len == 0 || a.hd == 0 || a.hd > 256 || a.hd % 8 != 0 || a.group == 0 || a.rows > 65535)
        return hipErrorInvalidValue;
    const size_t last = (size_t)a.len + a.rows - 1;
    if (last * a.ld * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    a.nsplit = (uint32_t)attn_splits(last);
    a.hchunks = (a.group + AT_HC - 1) / AT_HC;
    if (attn_rows_blocked(a.rows)) {
        // the matrix-core form: no partials, one launch
        if ((size_t)a.rows * a.heads * a.hd * 2 >= ((size_t)1 << 31)) return hipErrorInvalidValue;
        a.out = out;
        a.f16_out = f16_out ? 1u : 0u;
        const dim3 grid(((a.rows + AP_BR - 1) / AP_BR) * (a.heads / a.group) * a.hchunks);
        if (a.hd <= 64) hipLaunchKernelGGL(attn_rows_mfma<64>, grid, dim3(AP_T), 0, s, a);
        else if (a.hd <= 128) hipLaunchKernelGGL(attn_rows_mfma<128>, grid, dim3(AP_T), 0, s, a);
        else hipLaunchKernelGGL(attn_rows_mfma<256>, grid, dim3(AP_T), 0, s, a);
        return hipGetLastError();
    }
    const dim3 grid(a.nsplit, (a.heads / a.group) * a.hchunks, a.rows);
    if (a.hd <= 64) hipLaunchKernelGGL(attn_split<8>, grid, dim3(AT_T), 0, s, a);
    else if (a.hd <= 128) hipLaunchKernelGGL(attn_split<16>, grid, dim3(AT_T), 0, s, a);
    else hipLaunchKernelGGL(attn_split<32>, grid, dim3(AT_T), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 cgrid(a.heads, (a.hd + CM_D - 1) / CM_D, a.rows);
    if (f16_out)
        hipLaunchKernelGGL(attn_combine<true>, cgrid, dim3(CM_T), 0, s, a.po, a.pml, a.nsplit, a.len, a.heads,
                           a.hd, out);
    else
        hipLaunchKernelGGL(attn_combine<false>, cgrid, dim3(CM_T), 0, s, a.po, a.pml, a.nsplit, a.len, a.heads,
                           a.hd, out);
    return hipGetLastError();
}

hipError_t launch_qkv_rows(const QkvRowsArgs &a, hipStream_t s) {
    const uint32_t n = (a.heads + 2 * a.kv_heads) * a.hd;
    if (a.m == 0 || n == 0) return hipSuccess;
    if (a.m > 65535 || a.hd % 16 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(qkv_rows, dim3((n + 255) / 256, a.m), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_norm_rows(const float *x, const float *w, const float *b, size_t rows, size_t dim, float eps,
                            bool layer, uint16_t *y, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (rows > 0x7FFFFFFF || dim == 0) return hipErrorInvalidValue;
    if (layer)
        hipLaunchKernelGGL(norm_rows<true>, dim3((uint32_t)rows), dim3(MF_WAVES * 64), 0, s, x, w, b,
                           (uint32_t)dim, eps, y);
    else
        hipLaunchKernelGGL(norm_rows<false>, dim3((uint32_t)rows), dim3(MF_WAVES * 64), 0, s, x, w, b,
                           (uint32_t)dim, eps, y);
    return hipGetLastError();
}

hipError_t launch_round_q(const float *q, float scale, size_t count, uint16_t *qh, hipStream_t s) {
    hipLaunchKernelGGL(attn_round_q, dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, s, q, scale,
                       (uint32_t)count, qh);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float *x, const float *w, size_t rows, size_t dim, float eps, uint16_t *y,
                           hipStream_t s) {
    hipLaunchKernelGGL(rms_norm_rows, dim3((uint32_t)rows), dim3(MF_WAVES * 64), 0, s, x, w, (uint32_t)dim,
                       eps, y);
    return hipGetLastError();
}

hipError_t launch_glu(const uint16_t *both, size_t m, size_t n, uint32_t act, int tile8, uint16_t *y,
                      hipStream_t s) {
    const size_t total = m * n;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(glu_rows, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, s, both, (uint32_t)m,
                       (uint32_t)n, act, tile8, y);
    return hipGetLastError();
}

hipError_t launch_add_f16(const uint16_t *h, size_t count, float *y, hipStream_t s) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(add_f16_values, dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, s, h,
                       (uint64_t)count, y);
    return hipGetLastError();
}

}  // namespace smg
