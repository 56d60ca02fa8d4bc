// Host-side launch interface between the C ABI (api.hip) and the kernel
// translation units. Internal to the library.
#pragma once

#include <hip/hip_runtime.h>

#include "common.cuh"

namespace smg {

enum WKind { W_Q4 = 4, W_Q2 = 2, W_Q1 = 1, W_F16 = 16, W_BF16 = 17 };

// Device view of a weight set (layouts: common.cuh).
struct WDev {
    int kind;
    size_t n, k, block;
    size_t n_pad;     // columns padded to a multiple of 64
    size_t nchunks;   // chunks along K (Q4: 32 depths, Q2: 64, Q1: 128)
    size_t sc_rows;   // rows of the scale array
    const uint8_t *codes;   // Q4 nibbles / Q2 codes / Q1 signs
    const uint16_t *scales;
    const uint16_t *mins;   // Q4 affine only
    uint32_t codebook;      // Q2: the 4 int8 values, byte c = value of code c
    const uint16_t *dense;  // F16/BF16: [n_pad][k_pad] (column j's K contiguous)
    size_t k_pad;           // dense: K padded to a multiple of 64
};

// Rows at or below which the Q4 path runs the GEMV kernel; up to
// Q4_GEMV_WIDE_ROWS when the weights have one scale per 32-depth chunk (block
// >= 32) and k > 0, which the matrix-core GEMV serves with all 16 rows of its
// B operand (a 128-row GEMM tile would multiply mostly zero rows).
constexpr size_t Q4_GEMV_MAX_ROWS = 8;
constexpr size_t Q4_GEMV_WIDE_ROWS = 16;
inline bool q4_gemv_serves(const WDev &w, size_t m) {
    return m <= Q4_GEMV_MAX_ROWS || (m <= Q4_GEMV_WIDE_ROWS && w.block >= 32 && w.nchunks > 0);
}

// The Q4 GEMV for calls q4_gemv_serves() accepts; hipErrorNotSupported otherwise.
hipError_t launch_q4_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                          const EpArgs &ep, bool bf16, hipStream_t s);

// Progress words of a chained GEMV (device memory). Before each 4096-depth
// segment of A a workgroup waits, at most wait_ticks of the device wall clock,
// until *ready covers the segment; once every workgroup has stored its
// columns, the last one raises *done to done_value. sync[0] counts finished
// workgroups (zero before the call, zero again after it); sync[1] is set to 1
// when a wait timed out, and then *done is not raised.
struct ChainArgs {
    const unsigned long long *ready;  // or null: A complete at launch
    unsigned long long *done;         // or null
    unsigned int *sync;               // [2], set whenever ready or done is
    unsigned long long wait_ticks;
    unsigned long long done_value;
};

// The chained form of launch_q4_gemv for the MFMA GEMV's domain (f16,
// scale-only, block >= 32, k > 0, m <= Q4_GEMV_MAX_ROWS); hipErrorNotSupported
// outside it.
hipError_t launch_q4_gemv_chained(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                                  const EpArgs &ep, const ChainArgs &ch, hipStream_t s);

// Low-bit int8 path. scratch: device buffer of lowbit_scratch_bytes() bytes
// (used when the activations are quantized before the product kernel: several
// rows outside the persistent kernel, or blocks too large to quantize
// in-kernel). ep: the call's fused op-graph, which decides whether the
// persistent kernel serves (then 0); null sizes for the other kernels.
size_t lowbit_scratch_bytes(const WDev &w, size_t m, const EpArgs *ep = nullptr);
hipError_t launch_lowbit_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                              const EpArgs &ep, void *scratch, hipStream_t s);

// MFMA GEMM over any weight kind (Q4 / Q2 / Q1 dequantized to f16/bf16 in LDS,
// or dense), C[i,j] at dst[i*rs + j*cs] = ep(to16(beta * acc)).
// A graph of more than EP_FUSED nodes over an m x n C whose cells hold the
// product rounded to T (ep_tail, gemm_mfma.hip): src and dst may be the same
// array; add_dst adds alpha * old dst after the graph.
hipError_t launch_ep_tail(const uint16_t *src, long src_rs, long src_cs, uint16_t *dst, long dst_rs, long dst_cs,
                          size_t m, size_t n, float alpha, bool add_dst, const EpLong &ep, bool bf16, hipStream_t s);
hipError_t launch_gemm(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                       const uint16_t *lhs, long lhs_cs, long lhs_rs, float beta,
                       const EpArgs &ep, bool bf16, hipStream_t s, bool read_dst = false,
                       float alpha = 0.0f);
// Dense F16/BF16 weights ([n_pad][k_pad], column j's K contiguous, zero
// padded) from a k x n matrix B[l][j] = rhs[l*rhs_rs + j*rhs_cs].
hipError_t launch_pack_dense_strided(const uint16_t *rhs, long rhs_rs, long rhs_cs, size_t n, size_t k,
                                     size_t n_pad, size_t k_pad, uint16_t *dense, hipStream_t s);

// Q4 GEMM with register-resident weights (gemm_q4r.hip): f16 or bf16
// activations, block >= 32, K a multiple of 64, row-major 16-byte-aligned A.
// launch_gemm uses it whenever q4r_supported holds.
// With part (part_bytes of device memory, q4r_split_bytes(w, m) for the full
// split, untouched between the call and its kernels' completion) a grid too
// small to fill the device splits K into as many slices as part holds and
// adds them in a second kernel; with part null, or room for one slice, one
// kernel does all of K.
bool q4r_supported(const WDev &w, size_t m, long lhs_cs, long lhs_rs, const uint16_t *lhs, bool bf16);
size_t q4r_split_bytes(const WDev &w, size_t m);
hipError_t launch_q4r(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                      const uint16_t *lhs, long lhs_rs, float beta, const EpArgs &ep, float *part,
                      size_t part_bytes, bool bf16, hipStream_t s);
// The gate/up projection of a GatedLinear (w: Q4_0, 8 gate then 8 up columns
// a group, n = 16 * ceil(nh / 8)) with glu at the store: dst [m][nh] f16 holds
// glu(gate) * up from the rounded f16 projections, as launch_glu (tile8) gives
// from the GEMM's output. One kernel over all of K (split K has no gated
// reduce), so callers take it where q4r_split_bytes(w, m) is 0.
hipError_t launch_q4r_glu(const WDev &w, size_t m, uint16_t *dst, size_t nh, const uint16_t *lhs, uint32_t act,
                          hipStream_t s);
// y [m][n] f32 += the f16-rounded product of lhs and w (launch_q4r's store
// value, then the residual add), the add done in the split-K reduce: part
// holds q4r_split_bytes(w, m) bytes, which must be nonzero.
hipError_t launch_q4r_resid(const WDev &w, size_t m, const uint16_t *lhs, float *y, float *part, size_t part_bytes,
                            hipStream_t s);

// Compute units of the current device (cached per device).
int device_cus();

// Device-side repacks / dequant.
hipError_t launch_q4_dequant_dense(const WDev &q4, uint16_t *dense, bool to_bf16,
                                   hipStream_t s);

// dst[r][j] = (map[j] bit 30 ? src1 : src0)[r][map[j] & 0x3FFFFFFF], cells of
// cell_bytes (2, 16 or 64) in [rows][pad] grids (common.cuh's cell order);
// map[j] < 0 writes zeros.
hipError_t launch_gather_columns(void *dst, size_t dst_pad, const void *src0, const void *src1,
                                 size_t src_pad, const int32_t *map, size_t rows, size_t cell_bytes,
                                 hipStream_t s);

// ---- decode block (decode_block.hip) ---------------------------------------
// What the fused Q4 GEMVs of the decode block do at their source and store.
enum BlkStore : int {
    BS_RESID = 0,  // x[r][j] += f32(f16(result))        (Linear::accumulate)
    BS_GLU = 1,    // y[r][j] = f16(act(g) * u), device tiles of 8 gate + 8 up columns
    BS_QKV = 2     // RoPE'd q (scaled, f16) and the cache's new k / v row
};
struct BlkArgs {
    const float *nx, *nw;  // fused RMSNorm source: the f32 row and the norm's weights
    float eps;
    float *x;              // BS_RESID: [m][n] f32
    uint16_t *y;           // BS_GLU: [m][nh] f16
    uint32_t act, nh;      // BS_GLU: EP_ACT_SILU / EP_ACT_GELU, hidden width
    uint16_t *q_out;       // BS_QKV: [heads][hd] f16(q * scale)
    uint16_t *k_row, *v_row;  // BS_QKV: the cache rows at the new position
    const float *cs, *sn;  // BS_QKV: RoPE cos / sin at that position (null: no RoPE)
    float scale;           // BS_QKV: the score scale
    uint32_t heads, kv_heads, hd;
};
// A Q4 GEMV of m <= 8 rows (f16 `lhs`, or with norm the f32 row a.nx, m = 1,
// k <= 4096) with one of the stores above. Device column order: BS_QKV tiles
// are 8 columns of a head's first half and the same 8 of its second half;
// BS_GLU tiles 8 gate then the same 8 up columns.
hipError_t launch_blk_gemv(const WDev &w, size_t m, const uint16_t *lhs, const BlkArgs &a, int store,
                           bool norm, hipStream_t s);

// Attention of query rows over an f16 cache, split over keys. Row r (of
// rows, 1 for a decode step) attends to keys 0 .. len + r - 1: the causal
// prefix of a block of rows whose own keys are the cache's last rows.
struct AttnArgs {
    const uint16_t *q;       // [rows][heads][hd] f16(q * scale)
    const uint16_t *k, *v;   // [len + rows - 1][ld], KV head j at j*hd
    float *po;               // partial sums [rows][nsplit][heads][hd]
    float2 *pml;             // partial (max, sum) [rows][nsplit][heads]
    uint32_t len, ld, hd, heads, group;  // len: row 0's keys; group = heads / kv_heads
    uint32_t nsplit, hchunks;            // set by launch_attention (nsplit: the last row's)
    uint32_t rows;                       // 0 is taken as 1
    void *out;                           // set by launch_attention (the blocked form)
    uint32_t f16_out;                    // set by launch_attention (the blocked form)
};
// Blocks of this many rows run the matrix-core causal attention (one launch,
// no partials: po / pml unused); fewer rows run the split pass and merge,
// each row the same bits as a one-row call.
bool attn_rows_blocked(size_t rows);
size_t attn_splits(size_t len);
// Partial-sum bytes (po, then pml) launch_attention needs for `rows` rows whose
// last attends to `last_len` keys.
size_t attn_partial_floats(size_t rows, size_t last_len, size_t heads, size_t hd);
hipError_t launch_attention(const AttnArgs &a, void *out, bool f16_out, hipStream_t s);
// m rows of a qkv projection's f16 output (the device column order of the
// fused QKV store) to attention inputs at positions pos0 .. pos0 + m - 1:
// q and k rotated by NeoX RoPE (cs / sn: the table rows from position pos0,
// half = hd / 2 a row; null: no RoPE), q16 = f16(q * scale), k into k_cache
// and v into v_cache (the cache rows from pos0), as the fused store does.
struct QkvRowsArgs {
    const uint16_t *qkv;            // [m][(heads + 2 kv_heads) hd]
    uint16_t *q_out;                // [m][heads][hd]
    uint16_t *k_cache, *v_cache;    // [m][kv_heads hd]
    const float *cs, *sn;
    float scale;
    uint32_t m, heads, kv_heads, hd;
};
hipError_t launch_qkv_rows(const QkvRowsArgs &a, hipStream_t s);
// nn::layer_norm (bias may be null) or nn::rms_norm (layer = false) of f32 rows
// into f16.
hipError_t launch_norm_rows(const float *x, const float *w, const float *b, size_t rows, size_t dim, float eps,
                            bool layer, uint16_t *y, hipStream_t s);
hipError_t launch_round_q(const float *q, float scale, size_t count, uint16_t *qh, hipStream_t s);
hipError_t launch_rms_norm(const float *x, const float *w, size_t rows, size_t dim, float eps, uint16_t *y,
                           hipStream_t s);
// glu over m rows of 2n gate / up values: tile8 = 0, the reference's
// 32-column interleave; tile8 = 1, the device tiles of 8 gate + 8 up columns.
hipError_t launch_glu(const uint16_t *both, size_t m, size_t n, uint32_t act, int tile8, uint16_t *y,
                      hipStream_t s);
// y[i] += f32(h[i]) over count values (convert::add_f16).
hipError_t launch_add_f16(const uint16_t *h, size_t count, float *y, hipStream_t s);

// Measurement probes (probes.hip).
hipError_t launch_stream_read(const void *p, size_t bytes, unsigned *sink, hipStream_t s);
hipError_t launch_stream_read_store(const void *p, size_t bytes, uint16_t *out, size_t nout, hipStream_t s);
hipError_t launch_clock_probe(unsigned long long *out, unsigned iters, hipStream_t s);

// Sets the calling thread's smg_last_error() text and returns code.
int report(int code, const char *what);

}  // namespace smg
