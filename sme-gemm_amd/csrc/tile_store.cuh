// The GEMM kernels' output store: C = ep(to16(beta * acc)), shared by every
// prefill kernel. The caller rounds its accumulators to 16 bits into LDS, then
// walks its tile in groups of 8 consecutive columns of one row; each group is
// run through the op-graph on the rounded value (src/exec/macros.rs:188-206,
// the portable path's apply_ep_scalar order, src/exec/scalar.rs:58-140) and
// stored, 16 bytes at a time when the destination is row-major.
#pragma once

#include "common.cuh"

namespace smg {

struct StoreArgs {
    uint16_t *dst;
    long dst_rs, dst_cs;
    uint32_t m, n;
    float alpha;        // add_dst: C = T(graph result + alpha * old C)
    uint32_t add_dst;   // the SME epilogue's last step (csrc/epilogue.h:8-12)
};

// ROW / COL operand vectors of the graph, read once per tile into LDS as f32
// (colv [node][TBN], rowv [node][TBM]), so the cell loop touches global memory
// only for TENSOR operands. The caller puts a barrier between this and the
// first ep_store8.
template <bool BF16, int TBM, int TBN, int NT>
__device__ __forceinline__ void ep_load_vectors(const StoreArgs &g, const EpArgs &ep, float *colv,
                                                float *rowv, uint32_t row0, uint32_t col0) {
    const int t = threadIdx.x;
    for (uint32_t q = 0; q < ep.n_nodes; q++) {
        const uint32_t cls = ep.cls[q];
        const uint16_t *p = (const uint16_t *)ep.nodes[q].ptr;
        if (cls == EPC_COL)
            for (int c = t; c < TBN; c += NT) colv[q * TBN + c] = col0 + c < g.n ? to_f32<BF16>(p[col0 + c]) : 0.0f;
        if (cls == EPC_ROW)
            for (int r = t; r < TBM; r += NT) rowv[q * TBM + r] = row0 + r < g.m ? to_f32<BF16>(p[row0 + r]) : 0.0f;
    }
}

// Cells (rl, cl .. cl+7) of the tile (local coordinates), c8 their rounded
// 16-bit values.
template <bool BF16, int TBM, int TBN>
__device__ __forceinline__ void ep_store8(const StoreArgs &g, const EpArgs &ep, const float *colv,
                                          const float *rowv, uint4 c8, int rl, int cl, uint32_t row0,
                                          uint32_t col0) {
    const uint32_t row = row0 + rl, col = col0 + cl;
    if (row >= g.m || col >= g.n) return;
    const uint32_t ne = g.n - col < 8 ? g.n - col : 8;  // cells of this row group
    if (ep.n_nodes != 0) {
        uint32_t w4[4] = {c8.x, c8.y, c8.z, c8.w};
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = to_f32<BF16>((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
        for (uint32_t q = 0; q < ep.n_nodes; q++) {
            const EpNode &nd = ep.nodes[q];
            const uint32_t cls = ep.cls[q], fam = ep.fam[q];
            if (fam == EPF_ACT) {
                F8 y;
#pragma unroll
                for (int e = 0; e < 8; e++) y.v[e] = x[e];
                y = act8_fast(nd.aux, y, nd.scalar);
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = y.v[e];
                continue;
            }
            float v[8];
            if (cls == EPC_TENSOR) {
                // the 8 loads are issued together, then consumed
                const uint16_t *p = (const uint16_t *)nd.ptr + (size_t)row * (nd.ld == 0 ? g.n : nd.ld) + col;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (uint32_t)e < ne ? to_f32<BF16>(p[e]) : 0.0f;
            } else if (cls == EPC_COL) {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = colv[q * TBN + cl + e];
            } else {
                const float vs = cls == EPC_ROW ? rowv[q * TBM + rl] : nd.scalar;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = vs;
            }
            switch (fam) {  // uniform: one branch per node, then 8 lanes of arithmetic
#define SMG_EP_FAM(F)                                                           \
    case F:                                                                     \
        _Pragma("unroll") for (int e = 0; e < 8; e++) x[e] = ep_arith(F, x[e], v[e]); \
        break;
                SMG_EP_FAM(EPF_ADD) SMG_EP_FAM(EPF_MUL) SMG_EP_FAM(EPF_SUB)
                SMG_EP_FAM(EPF_DIV) SMG_EP_FAM(EPF_MAX) SMG_EP_FAM(EPF_MIN)
#undef SMG_EP_FAM
            default: break;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
            w4[e] = (uint32_t)from_f32<BF16>(x[2 * e]) | ((uint32_t)from_f32<BF16>(x[2 * e + 1]) << 16);
        c8 = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
    uint16_t *dp = g.dst + (size_t)row * g.dst_rs + (size_t)col * g.dst_cs;
    if (g.add_dst) {
        uint32_t w4[4] = {c8.x, c8.y, c8.z, c8.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if ((uint32_t)e >= ne) break;
            const float x = to_f32<BF16>((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
            const uint16_t y = from_f32<BF16>(x + g.alpha * to_f32<BF16>(dp[(size_t)e * g.dst_cs]));
            w4[e / 2] = (w4[e / 2] & (0xFFFF0000u >> (16 * (e % 2)))) | ((uint32_t)y << (16 * (e % 2)));
        }
        c8 = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
    if (g.dst_cs == 1 && ne == 8 && ((uintptr_t)dp & 15) == 0) {
        *(uint4 *)dp = c8;
        return;
    }
    const uint32_t w4[4] = {c8.x, c8.y, c8.z, c8.w};
    for (uint32_t e = 0; e < ne; e++) dp[(size_t)e * g.dst_cs] = (uint16_t)(w4[e / 2] >> (16 * (e % 2)));
}

// An activation over R x 8 cells: the logistic kinds inline (no call), one
// loop per kind (as act_f32_fast: silu x*L(x), sigmoid L(x), tanh-gelu
// x*L(2u)); the rest one act8_fast call per row.
template <int R>
__device__ __forceinline__ void act_rows(uint32_t aux, float alpha, F8 (&x)[R]) {
    if (aux == 3) {
#pragma unroll
        for (int j = 0; j < R; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) x[j].v[e] = mul_logistic(x[j].v[e], x[j].v[e]);
    } else if (aux == 5) {
#pragma unroll
        for (int j = 0; j < R; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) x[j].v[e] = mul_logistic(1.0f, x[j].v[e]);
    } else if (aux == 2) {
#pragma unroll
        for (int j = 0; j < R; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = x[j].v[e];
                x[j].v[e] = mul_logistic(v, 2.0f * 0.7978845608028654f * (v + 0.044715f * v * v * v));
            }
    } else if (aux != EP_ACT_NONE) {
#pragma unroll
        for (int j = 0; j < R; j++) x[j] = act8_fast(aux, x[j], alpha);
    }
}

// R rows (rl0 + rstep * j) x the same 8 columns (cl .. cl+7) of the tile:
// what one thread stores when the tile's column groups divide the thread count.
// The staged 16-bit values are read from tile (row stride cs halfs); a COL
// operand is read once for all R rows, and every node runs over the R x 8 cells
// before the next, so the R rows' work overlaps.
template <bool BF16, int TBM, int TBN, int R>
__device__ __forceinline__ void ep_store_rows(const StoreArgs &g, const EpArgs &ep, const float *colv,
                                              const float *rowv, const uint16_t *tile, int cs, int rl0,
                                              int rstep, int cl, uint32_t row0, uint32_t col0) {
    const uint32_t col = col0 + cl;
    if (col >= g.n) return;
    const uint32_t ne = g.n - col < 8 ? g.n - col : 8;
    uint4 c8[R];
#pragma unroll
    for (int j = 0; j < R; j++) c8[j] = *(const uint4 *)(tile + (rl0 + rstep * j) * cs + cl);
    if (ep.n_nodes != 0) {
        F8 x[R];
#pragma unroll
        for (int j = 0; j < R; j++) {
            const uint32_t w4[4] = {c8[j].x, c8[j].y, c8[j].z, c8[j].w};
#pragma unroll
            for (int e = 0; e < 8; e++) x[j].v[e] = to_f32<BF16>((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
        }
        for (uint32_t q = 0; q < ep.n_nodes; q++) {
            const EpNode &nd = ep.nodes[q];
            const uint32_t cls = ep.cls[q], fam = ep.fam[q];
            if (fam == EPF_ACT) {
                act_rows<R>(nd.aux, nd.scalar, x);
                continue;
            }
            if (cls == EPC_TENSOR) {
                const size_t ld = nd.ld == 0 ? g.n : nd.ld;
#pragma unroll
                for (int j = 0; j < R; j++) {
                    const uint32_t row = row0 + rl0 + rstep * j;
                    const uint16_t *p = (const uint16_t *)nd.ptr + (size_t)(row < g.m ? row : 0) * ld + col;
                    float v[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = (uint32_t)e < ne ? to_f32<BF16>(p[e]) : 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; e++) x[j].v[e] = ep_arith(fam, x[j].v[e], v[e]);
                }
                continue;
            }
            float v[R][8];
            if (cls == EPC_COL) {
                float cv[8];
#pragma unroll
                for (int e = 0; e < 8; e++) cv[e] = colv[q * TBN + cl + e];
#pragma unroll
                for (int j = 0; j < R; j++)
#pragma unroll
                    for (int e = 0; e < 8; e++) v[j][e] = cv[e];
            } else {
#pragma unroll
                for (int j = 0; j < R; j++) {
                    const float vs = cls == EPC_ROW ? rowv[q * TBM + rl0 + rstep * j] : nd.scalar;
#pragma unroll
                    for (int e = 0; e < 8; e++) v[j][e] = vs;
                }
            }
            switch (fam) {  // uniform: one branch per node, then R x 8 lanes of arithmetic
#define SMG_EP_FAM(F)                                                                              \
    case F:                                                                                        \
        _Pragma("unroll") for (int j = 0; j < R; j++) _Pragma("unroll") for (int e = 0; e < 8; e++) \
            x[j].v[e] = ep_arith(F, x[j].v[e], v[j][e]);                                            \
        break;
                SMG_EP_FAM(EPF_ADD) SMG_EP_FAM(EPF_MUL) SMG_EP_FAM(EPF_SUB)
                SMG_EP_FAM(EPF_DIV) SMG_EP_FAM(EPF_MAX) SMG_EP_FAM(EPF_MIN)
#undef SMG_EP_FAM
            default: break;
            }
        }
#pragma unroll
        for (int j = 0; j < R; j++) {
            uint32_t w4[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                w4[e] = (uint32_t)from_f32<BF16>(x[j].v[2 * e]) | ((uint32_t)from_f32<BF16>(x[j].v[2 * e + 1]) << 16);
            c8[j] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    }
#pragma unroll
    for (int j = 0; j < R; j++) {
        const uint32_t row = row0 + rl0 + rstep * j;
        if (row >= g.m) continue;
        uint16_t *dp = g.dst + (size_t)row * g.dst_rs + (size_t)col * g.dst_cs;
        if (g.dst_cs == 1 && ne == 8 && ((uintptr_t)dp & 15) == 0) {
            *(uint4 *)dp = c8[j];
            continue;
        }
        const uint32_t w4[4] = {c8[j].x, c8[j].y, c8[j].z, c8[j].w};
        for (uint32_t e = 0; e < ne; e++) dp[(size_t)e * g.dst_cs] = (uint16_t)(w4[e / 2] >> (16 * (e % 2)));
    }
}

// The 8 column operand values (col .. col+7) of a compiled store, as 16-bit
// patterns, read before the tile is staged so that their latency overlaps the
// accumulator exchange; columns past n read zero (never stored).
struct EpCols {
    uint16_t a[8], b[8];
};
template <int EPV>
__device__ __forceinline__ void ep_cols_load(const uint16_t *col_a, const uint16_t *col_b, uint32_t col,
                                             uint32_t n, EpCols &cv) {
    if constexpr (EPV >= 2) {
        const rsrc_t rb = make_rsrc(col_b, n * 2u);
#pragma unroll
        for (int e = 0; e < 8; e++) cv.b[e] = bload2(rb, col + e < n ? (col + e) * 2u : OOB);
    }
    if constexpr (EPV == 3) {
        const rsrc_t ra = make_rsrc(col_a, n * 2u);
#pragma unroll
        for (int e = 0; e < 8; e++) cv.a[e] = bload2(ra, col + e < n ? (col + e) * 2u : OOB);
    }
}

// ep_store_rows compiled for the common graphs (EpPick's v = EPV: 1 none, 2
// [add_col] + act, 3 [mul_col, add_col] + act; add_dst must be 0): the same
// f32 steps in the same order on the rounded value -- x * a, then + b, then
// the activation as act_rows -- without the per-node interpretation, whose
// code (every family and class, unrolled over R x 8 cells) is what a tile's
// store otherwise spends its time fetching and branching through.
template <bool BF16, int R, int EPV>
__device__ __forceinline__ void ep_store_rows_c(const StoreArgs &g, uint32_t act, float alpha, const EpCols &cv,
                                                const uint16_t *tile, int cs, int rl0, int rstep, int cl,
                                                uint32_t row0, uint32_t col0) {
    const uint32_t col = col0 + cl;
    if (col >= g.n) return;
    const uint32_t ne = g.n - col < 8 ? g.n - col : 8;
    uint4 c8[R];
#pragma unroll
    for (int j = 0; j < R; j++) c8[j] = *(const uint4 *)(tile + (rl0 + rstep * j) * cs + cl);
    if constexpr (EPV >= 2) {
        float va[8], vb[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            va[e] = to_f32<BF16>(cv.a[e]);
            vb[e] = to_f32<BF16>(cv.b[e]);
        }
        F8 x[R];
#pragma unroll
        for (int j = 0; j < R; j++) {
            const uint32_t w4[4] = {c8[j].x, c8[j].y, c8[j].z, c8[j].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float v = to_f32<BF16>((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
                if constexpr (EPV == 3) v = v * va[e];
                x[j].v[e] = v + vb[e];
            }
        }
        act_rows<R>(act, alpha, x);
#pragma unroll
        for (int j = 0; j < R; j++) {
            uint32_t w4[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                w4[e] = (uint32_t)from_f32<BF16>(x[j].v[2 * e]) | ((uint32_t)from_f32<BF16>(x[j].v[2 * e + 1]) << 16);
            c8[j] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    }
#pragma unroll
    for (int j = 0; j < R; j++) {
        const uint32_t row = row0 + rl0 + rstep * j;
        if (row >= g.m) continue;
        uint16_t *dp = g.dst + (size_t)row * g.dst_rs + (size_t)col * g.dst_cs;
        if (g.dst_cs == 1 && ne == 8 && ((uintptr_t)dp & 15) == 0) {
            *(uint4 *)dp = c8[j];
            continue;
        }
        const uint32_t w4[4] = {c8[j].x, c8[j].y, c8[j].z, c8[j].w};
        for (uint32_t e = 0; e < ne; e++) dp[(size_t)e * g.dst_cs] = (uint16_t)(w4[e / 2] >> (16 * (e % 2)));
    }
}

// The gated store (f16 only): the tile's columns come in groups of 8 gate and
// 8 up values (the device layout of a GatedLinear's gate/up weights), and the
// store writes glu(gate) * up for each pair -- glu_rows' tile8 arithmetic on
// the same rounded f16 values -- to column (col0 + cu) / 2 + e of g.dst, which
// holds hidden = nh columns. cu: the gate group's column in the tile (a
// multiple of 16).
template <int R>
__device__ __forceinline__ void ep_store_glu8(const StoreArgs &g, uint32_t act, uint32_t nh, const uint16_t *tile,
                                              int cs, int rl0, int rstep, int cu, uint32_t row0, uint32_t col0) {
    const uint32_t col = (col0 + cu) / 2;
    if (col >= nh) return;
    const uint32_t ne = nh - col < 8 ? nh - col : 8;
#pragma unroll
    for (int j = 0; j < R; j++) {
        const uint32_t row = row0 + rl0 + rstep * j;
        if (row >= g.m) continue;
        const uint16_t *tr = tile + (rl0 + rstep * j) * cs + cu;
        const uint4 gq = *(const uint4 *)tr, uq = *(const uint4 *)(tr + 8);
        const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w}, uw[4] = {uq.x, uq.y, uq.z, uq.w};
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint32_t h2 = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float gv = f16_to_f32((uint16_t)(gw[e] >> (16 * h)));
                const float uv = f16_to_f32((uint16_t)(uw[e] >> (16 * h)));
                h2 |= (uint32_t)f32_to_f16(glu_act(act, gv) * uv) << (16 * h);
            }
            w4[e] = h2;
        }
        uint16_t *dp = g.dst + (size_t)row * g.dst_rs + col;
        if (ne == 8 && ((uintptr_t)dp & 15) == 0) {
            *(uint4 *)dp = make_uint4(w4[0], w4[1], w4[2], w4[3]);
            continue;
        }
        for (uint32_t e = 0; e < ne; e++) dp[e] = (uint16_t)(w4[e / 2] >> (16 * (e % 2)));
    }
}

}  // namespace smg
