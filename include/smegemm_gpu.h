/*
 * smegemm_gpu.h -- C ABI of the MI355X (gfx950) quantized-weight matmul
 * library. It replaces the reference crate's FFI for this path
 * (src/ffi.rs <-> csrc/sme_gemm_api.h) and the kernel dispatch in
 * src/kernels/q4/matmul.rs and src/kernels/lowbit/matmul.rs.
 *
 * Conventions (the reference's, csrc/sme_gemm_api.h and ARCHITECTURE.md):
 *   - f16 / bf16 values travel as uint16_t bit patterns.
 *   - Every entry point returns int: 0 = done; non-zero = failed with the
 *     output untouched (the reference's rc contract, src/kernels/q4/matmul.rs:85-90),
 *     so the caller may fall back. Codes below say why.
 *   - `ep == NULL` (or n_nodes == 0) means no epilogue. A trailing activation
 *     is the last node with op EP_OP_ACT, as resolve_nodes builds it
 *     (src/exec/scalar.rs:28-53).
 *   - Host-pointer entry points (gemm_gpu_*) are synchronous, like the
 *     reference: dst is fully written on return. Epilogue operand pointers
 *     are host pointers there.
 *   - Device-pointer entry points (smg_*_dev) are asynchronous on `stream`
 *     (a hipStream_t, NULL = the null stream); lhs, dst and every epilogue
 *     operand pointer are device pointers (memory the weights' GPU can read:
 *     its device memory, managed or pinned host memory -- anything else is
 *     refused with SMG_EINVAL, except while the stream is being captured).
 *   - Safe for concurrent callers on different host threads: each thread gets
 *     its own stream and staging buffers for the host-pointer entry points.
 *
 * Weights live on the device behind an opaque handle (the "prepack"): the
 * reference keeps them in Q4Weights / Q2Weights / Q1Weights / Packed<f16>,
 * and a Rust binding keeps the handle in those types (it owns one and calls
 * smg_weights_destroy when they drop).
 */
#ifndef SMEGEMM_GPU_H
#define SMEGEMM_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- return codes --------------------------------------------------------- */
#define SMG_OK 0
#define SMG_EINVAL -1  /* bad argument (e.g. block not a power of two); the reference's -1 */
#define SMG_ENOMEM -2  /* device allocation failed */
#define SMG_EHIP -3    /* a HIP runtime call or launch failed */
#define SMG_ENODEV -4  /* no usable gfx950 device */
#define SMG_EKIND -5   /* weight handle of the wrong kind for this entry point */

/* Test hook: while the environment holds SMG_TEST_FAIL_ALLOC=1 (read at each
 * attempt) every device allocation the library makes fails, so the call
 * returns SMG_ENOMEM before writing dst -- the contract the reference's
 * callers rely on to take their portable path on a non-zero return
 * (src/kernels/q4/matmul.rs:85-89). Buffers a call allocated earlier
 * (the host-call staging area, the device-form scratch pool) are kept and
 * reused, so only a first allocation or a growth fails. */

/* ---- epilogue ABI: byte-identical to csrc/epilogue.h:136-236 -------------- */
enum ep_act {
    EP_ACT_NONE = 0, EP_ACT_RELU = 1, EP_ACT_GELU = 2, EP_ACT_SILU = 3, EP_ACT_TANH = 4,
    EP_ACT_SIGMOID = 5, EP_ACT_LEAKY_RELU = 6, EP_ACT_RELU6 = 7, EP_ACT_HARDSIGMOID = 8,
    EP_ACT_HARDSWISH = 9, EP_ACT_ABS = 10, EP_ACT_NEG = 11, EP_ACT_SQUARE = 12,
    EP_ACT_SIGN = 13, EP_ACT_SQRT = 14, EP_ACT_SOFTSIGN = 15, EP_ACT_RECIP = 16,
    EP_ACT_RSQRT = 17, EP_ACT_EXP = 18, EP_ACT_LOG = 19, EP_ACT_ELU = 20, EP_ACT_SELU = 21,
    EP_ACT_SOFTPLUS = 22, EP_ACT_MISH = 23, EP_ACT_GELU_EXACT = 24
};

enum ep_op {
    EP_OP_ADD_SCALAR = 0, EP_OP_MUL_SCALAR = 1, EP_OP_ADD_ROW = 2, EP_OP_MUL_ROW = 3,
    EP_OP_ADD_COL = 4, EP_OP_MUL_COL = 5, EP_OP_ADD_TENSOR = 6, EP_OP_MUL_TENSOR = 7,
    EP_OP_ACT = 8, EP_OP_MAX_SCALAR = 9, EP_OP_MIN_SCALAR = 10, EP_OP_SUB_SCALAR = 11,
    EP_OP_SUB_ROW = 12, EP_OP_SUB_COL = 13, EP_OP_SUB_TENSOR = 14, EP_OP_DIV_SCALAR = 15,
    EP_OP_DIV_ROW = 16, EP_OP_DIV_COL = 17, EP_OP_DIV_TENSOR = 18, EP_OP_MAX_ROW = 19,
    EP_OP_MAX_COL = 20, EP_OP_MAX_TENSOR = 21, EP_OP_MIN_ROW = 22, EP_OP_MIN_COL = 23,
    EP_OP_MIN_TENSOR = 24
};

/* One op-graph node (csrc/epilogue.h:214-221; Rust mirror src/epilogue/mod.rs:150). */
typedef struct {
    uint32_t op;     /* enum ep_op */
    uint32_t aux;    /* enum ep_act for EP_OP_ACT */
    float scalar;    /* *_SCALAR operand; alpha of LEAKY_RELU / ELU */
    const void *ptr; /* ROW (m) / COL (n) / TENSOR (rows at stride ld) operand, f16 or bf16 */
    size_t ld;       /* TENSOR row stride in elements; 0 = n */
} EpNode;

/* csrc/epilogue.h:233-236 */
typedef struct {
    uint32_t n_nodes;
    const EpNode *nodes;
} ep_desc16;

/* Nodes one call carries to the device (by value, in the kernel arguments).
 * Up to SMG_FUSED_EP_NODES run in the product kernel's store; a longer graph
 * runs as a second pass over C that reads each stored cell (the product
 * rounded to T) and applies the whole graph -- the reference's own order,
 * GEMM to T then apply_ep_scalar (src/exec/macros.rs:188-206), so the
 * results are the same. Longer than SMG_MAX_EP_NODES returns SMG_EINVAL, as
 * does a graph longer than SMG_FUSED_EP_NODES on the chained GEMV (its done
 * flag is raised by the product kernel itself). */
#define SMG_FUSED_EP_NODES 16
#define SMG_MAX_EP_NODES 64

/* The checks every entry point makes of an epilogue before any device work,
 * for an output n columns wide: at most SMG_MAX_EP_NODES nodes, known ops and
 * activations, a non-NULL operand pointer on every ROW / COL / TENSOR node, a
 * TENSOR row stride of 0 or >= n. 0 or SMG_EINVAL (reason in smg_last_error).
 * Operand lengths are the caller's to check, as validate_ep does on the Rust
 * side (src/exec/guard.rs:112-147). */
int smg_ep_check(const ep_desc16 *ep, size_t n);

/* ---- weight handles ------------------------------------------------------- */
typedef struct smg_weights smg_weights;

/* Q4: replaces Q4Weights::new / with_params (src/kernels/q4/weights.rs:50-123).
 * Row-major input: weight idx = d*n + j is nibble idx%2 (low first) of byte
 * idx/2, code = nib < 8 ? nib : nib - 16; scales[j*ceil(k/block) + d/block]
 * (f16); mins the same shape or NULL (Q4Form::Scale). block: a power of two. */
int smg_q4_create(const uint8_t *quants, const uint16_t *scales, const uint16_t *mins, size_t n,
                  size_t k, size_t block, smg_weights **out);

/* Q4 from the reference's band-major resident arrays -- exactly what src/ffi.rs
 * passes to gemm_sme_f16f16_q4 (nibbles/scales/mins of Q4Weights,
 * weights.rs:89-113): 128-column bands, 64 bytes per depth, scales [band][blk][128]. */
int smg_q4_create_band(const uint8_t *nibbles, const uint16_t *scales, const uint16_t *mins,
                       size_t n, size_t k, size_t block, smg_weights **out);

/* Q2: replaces Q2Weights::new (src/kernels/lowbit/q2.rs:53-86). Row-major codes,
 * weight idx = d*n + j at bits 2*(idx%4) of byte idx/4; scales[j*nbk + d/block];
 * codebook: the 4 int8 values (Q2Params, lowbit/mod.rs:38-94).
 * block: power of two in [16, 65536]. */
int smg_q2_create(const uint8_t *codes, const uint16_t *scales, const int8_t *codebook,
                  size_t n, size_t k, size_t block, smg_weights **out);
/* Q2 from the band-major arrays src/ffi.rs passes (q2.rs:12-20,148-161). */
int smg_q2_create_band(const uint8_t *codes, const uint16_t *scales, const int8_t *codebook,
                       size_t n, size_t k, size_t block, smg_weights **out);

/* Q1: replaces Q1Weights::new (src/kernels/lowbit/q1.rs:47-107). layout 0 =
 * WeightLayout::OutIn (idx = j*k + d), 1 = InOut (idx = d*n + j); bit idx%8 of
 * byte idx/8, set = +scale. */
int smg_q1_create(const uint8_t *signs, const uint16_t *scales, int layout, size_t n, size_t k,
                  size_t block, smg_weights **out);
/* Q1 from the band-major arrays src/ffi.rs passes (q1.rs:186-201). */
int smg_q1_create_band(const uint8_t *signs, const uint16_t *scales, size_t n, size_t k,
                       size_t block, smg_weights **out);

/* Load-time quantizers (host code): f32 weights w (n outputs x k inputs;
 * layout 0 = WeightLayout::OutIn, w[j*k + d]; 1 = InOut, w[d*n + j]) to the
 * row-major input arrays the create functions above take. The caller owns the
 * outputs: quants ceil(k*n/2) bytes, codes ceil(k*n/4), signs ceil(k*n/8)
 * (OutIn, as Q1Weights::quantize packs them), scales / mins n*ceil(k/block)
 * f16. Replace Q4Weights::quantize (src/kernels/q4/quantize.rs:29-81; affine
 * 1 = Q4Form::Affine, else mins may be NULL), Q2Weights::quantize
 * (src/kernels/lowbit/q2.rs:110-143; SMG_EINVAL for an all-zero codebook) and
 * Q1Weights::quantize (src/kernels/lowbit/q1.rs:116-147). */
int smg_q4_quantize(const float *w, int layout, size_t n, size_t k, size_t block, int affine,
                    uint8_t *quants, uint16_t *scales, uint16_t *mins);
int smg_q2_quantize(const float *w, int layout, size_t n, size_t k, size_t block,
                    const int8_t *codebook, uint8_t *codes, uint16_t *scales);
int smg_q1_quantize(const float *w, int layout, size_t n, size_t k, size_t block, uint8_t *signs,
                    uint16_t *scales);

/* Dense Packed<f16> / Packed<bf16>: replaces prepack_f16 / prepack_bf16
 * (src/kernels/f16.rs:212; bf16.rs:240) and gemm_sme_f16f16_packb
 * (csrc/sme_gemm_api.h:94). B[l][j] = rhs[l*rhs_rs + j*rhs_cs] (k x n). */
int smg_f16_prepack(const uint16_t *rhs, size_t n, size_t k, long rhs_rs, long rhs_cs,
                    smg_weights **out);
int smg_bf16_prepack(const uint16_t *rhs, size_t n, size_t k, long rhs_rs, long rhs_cs,
                     smg_weights **out);

/* Eager dequant of a Q4 handle to a dense handle on the device: replaces
 * dequant_q4 / dequant_q4_with (f16: one RNE rounding of scale*code+min) and
 * dequant_q4_bf16 / _with (bf16 through f32), src/kernels/q4/mod.rs:145-257. */
int smg_q4_dequant(const smg_weights *q4, int to_bf16, smg_weights **out);

/* Column repacks on the device (exact: codes, scales and mins move unchanged).
 * smg_q4_permute_columns: output column j is column perm[j] of q4 (perm holds
 * n entries < n); replaces Q4Weights::permute_columns
 * (src/kernels/q4/weights.rs:125-163). smg_q1_interleave: gate and up (same n,
 * k, block) to 2n columns, each 32-column chunk of gate followed by the same
 * chunk of up; replaces Q1Weights::interleave (src/kernels/lowbit/q1.rs:146-185). */
int smg_q4_permute_columns(const smg_weights *q4, const size_t *perm, smg_weights **out);
/* smg_q1_interleave for Q4 (same n, k, block and form): the weights
 * GatedLinear::quantize builds (src/linear.rs:601-619, 656-671), exactly, from
 * the gate and up weights quantized on their own (Q4 blocks run along K, so a
 * column's codes and scales do not depend on its neighbours). */
int smg_q4_interleave(const smg_weights *gate, const smg_weights *up, smg_weights **out);
int smg_q1_interleave(const smg_weights *gate, const smg_weights *up, smg_weights **out);

/* A second device copy of a handle's weights (device-to-device; no host
 * repack). Used to rotate benchmark weights past the 256 MB MALL. */
int smg_weights_clone(const smg_weights *w, smg_weights **out);

void smg_weights_destroy(smg_weights *w);
/* n, k, block (0 for dense) and device bytes of a handle. */
int smg_weights_info(const smg_weights *w, size_t *n, size_t *k, size_t *block, size_t *bytes);
/* The HIP device ordinal a handle's weights live on (where its calls run). */
int smg_weights_device(const smg_weights *w, int *device);

/* ---- host-pointer drop-ins (synchronous) ---------------------------------- */

/* matmul_q4 / matmul_q4_ep: C = ep(A @ dequant(B)); replaces gemm_sme_f16f16_q4
 * (csrc/sme_gemm_api.h:97-99). lhs m x k f16 row-major, dst m x n f16. */
int gemm_gpu_f16f16_q4(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep);
/* matmul_q4_bf16 / _ep; replaces gemm_sme_b16b16_q4 (csrc/sme_gemm_api.h:66-69). */
int gemm_gpu_b16b16_q4(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep);
/* matmul_q2 / _ep and matmul_q1 / _ep (int8 path, bit-exact with
 * src/kernels/lowbit/matmul.rs:376-398); replace gemm_sme_f16_q2 / _q1
 * (csrc/sme_gemm_api.h:208-213). The handle's kind selects Q2 or Q1. */
int gemm_gpu_f16_q2(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                    const ep_desc16 *ep);
int gemm_gpu_f16_q1(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                    const ep_desc16 *ep);
/* matmul_q2_mopa / matmul_q1_mopa (+_ep): f16 weights scale*value rounded once,
 * f16 activations, f32 accumulation; replace gemm_sme_f16f16_q2 / _q1
 * (csrc/sme_gemm_api.h:110-115). */
int gemm_gpu_f16f16_q2(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep);
int gemm_gpu_f16f16_q1(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep);
/* The dense packed GEMM behind Gemm::new(&a, &packed, m)...run(&mut c) and
 * matmul_f16_packed: replaces gemm_sme_f16f16_run_packed
 * (csrc/sme_gemm_api.h:120-123). C[i,j] at dst[i*dst_rs + j*dst_cs];
 * A[i,l] at lhs[i*lhs_rs + l*lhs_cs]; dst = ep(beta * A@B) (read_dst == 0,
 * the only form the reference's callers use, src/exec/macros.rs:131-150;
 * alpha_bits is then ignored). read_dst != 0: with no op-graph,
 * dst = T(alpha * dst + beta * A@B), one rounding (src/reference.rs:349-387);
 * with a graph, dst = T(graph result + alpha * dst), the SME epilogue's order
 * (csrc/epilogue.h:8-12). */
int gemm_gpu_f16f16_run_packed(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs,
                               long dst_rs, int read_dst, const uint16_t *lhs, long lhs_cs,
                               long lhs_rs, const smg_weights *b_pack, uint16_t alpha_bits,
                               uint16_t beta_bits, const ep_desc16 *ep);
int gemm_gpu_b16b16_run_packed(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs,
                               long dst_rs, int read_dst, const uint16_t *lhs, long lhs_cs,
                               long lhs_rs, const smg_weights *b_pack, uint16_t alpha_bits,
                               uint16_t beta_bits, const ep_desc16 *ep);
/* Strided unpacked dense GEMM, C = alpha*C + beta*(A @ B) (gemm_f16 /
 * matmul_f16, src/kernels/f16.rs:89-204; gemm_bf16 / matmul_bf16,
 * src/kernels/bf16.rs:101-200): replace gemm_sme_f16f16_run
 * (csrc/sme_gemm_api.h:116-119), gemm_sme_f16f32_run (:84-87),
 * gemm_sme_b16b16_run (:70-73) and gemm_sme_bf16f32_run (:80-83). Host
 * pointers; C[i,j] at dst[i*dst_rs + j*dst_cs], A[i,l] at
 * lhs[i*lhs_rs + l*lhs_cs], B[l,j] at rhs[l*rhs_rs + j*rhs_cs]. Strides are
 * non-negative; A and B may repeat cells (a zero stride), C's cells must be
 * distinct with nested strides (dst_rs >= n*dst_cs or dst_cs >= m*dst_rs; a
 * single row or column needs only a positive stride), else SMG_EINVAL -- its
 * cells are written in parallel. C is read only when read_dst != 0; then
 * dst = T(alpha * dst + beta * acc) with one rounding. All four accumulate in
 * f32, as the portable path they fall back to (src/reference.rs:308-387).
 * B is packed on the device for the call. */
int gemm_gpu_f16f16_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs,
                        int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                        const uint16_t *rhs, long rhs_cs, long rhs_rs, uint16_t alpha_bits,
                        uint16_t beta_bits);
int gemm_gpu_f16f32_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs,
                        int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                        const uint16_t *rhs, long rhs_cs, long rhs_rs, uint16_t alpha_bits,
                        uint16_t beta_bits);
int gemm_gpu_b16b16_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs,
                        int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                        const uint16_t *rhs, long rhs_cs, long rhs_rs, uint16_t alpha_bits,
                        uint16_t beta_bits);
int gemm_gpu_bf16f32_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs,
                         int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                         const uint16_t *rhs, long rhs_cs, long rhs_rs, uint16_t alpha_bits,
                         uint16_t beta_bits);
/* The same on device pointers, enqueued on `stream` (bf16 != 0: bf16 operands);
 * B is packed into a scratch buffer of the stream's own (grow-only, kept). */
int smg_gemm_run_dev(int bf16, size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs,
                     int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs, const uint16_t *rhs,
                     long rhs_cs, long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits, void *stream);

/* Whether an m-row Q4 call runs the GEMV kernel whatever the weights' block
 * (m <= 8; replaces gemm_sme_f16f16_q4_single, csrc/sme_gemm_api.h:107).
 * Weights with a block of 32 or more also take the GEMV up to 32 rows (one
 * launch per 16 rows), which this query, given no block, does not report. */
int gemm_gpu_f16f16_q4_single(size_t m, size_t n, size_t k);
/* One link of a chain (q4_chained, src/kernels/q4/matmul.rs:116-164); replaces
 * gemm_sme_f16f16_q4_chained (csrc/sme_gemm_api.h:102-105). done / ready are
 * the reference's std::atomic<size_t> words (either NULL), written and read by
 * other host threads: the call reads A only once *ready (acquire) covers all
 * k depths, computes as gemm_gpu_f16f16_q4 (the whole op-graph in the kernel,
 * the same bits), and raises *done (release) to n once C is stored. */
int gemm_gpu_f16f16_q4_chained(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                               const ep_desc16 *ep, size_t *done, const size_t *ready);

/* ---- device-pointer entry points (asynchronous on `stream`) --------------- */
int smg_q4_matmul_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                      const ep_desc16 *ep, int bf16, void *stream);
/* The chained link between kernels on the device (the GPU form of
 * gemm_sme_f16f16_q4_chained, csrc/sme_gemm_api.h:102-105, for the decode
 * GEMV: f16, scale-only Q4, block >= 32, k > 0, 1 <= m <= 8; SMG_EINVAL
 * otherwise). ready / done are device words (either NULL) counting depths of A
 * and columns of C: each workgroup first issues its weight loads, then waits
 * until *ready covers the 4096-depth segment of A it reads next, and once
 * every workgroup has stored its columns the last one raises *done to n
 * (release; all columns form one pass). A producer kernel on another stream
 * raises *ready with a release store. sync (needed when done or ready is
 * set): two device words, zero before the first call; sync[0] is zero again
 * after each call, sync[1] becomes 1 if
 * a wait lasted wait_us (0: 100 ms) without *ready covering its segment, and
 * then *done is not raised and the columns of the workgroups that timed out
 * are not stored. Chains that run at once each need their own sync words. */
int smg_q4_chained_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep, unsigned long long *done, const unsigned long long *ready,
                       unsigned int *sync, unsigned int wait_us, void *stream);
int smg_lowbit_matmul_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                          const ep_desc16 *ep, void *stream);
/* smg_lowbit_matmul_dev that allocates nothing. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). Same
 * arguments, bits and stream semantics; the quantized activations of a
 * multi-row call (q, block scales and sums: m*K bytes and a little more) are
 * staged in a static device array of this library, SMG_NOALLOC_SCRATCH_BYTES
 * per device and held by each device until the process ends, instead of an
 * allocated buffer. A call needing more returns SMG_EINVAL with nothing
 * enqueued. Every call on one device shares that array and each call rewrites
 * what it reads: calls that overlap on one GPU (on different streams, or on
 * one stream from several threads) race on it. */
#define SMG_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)
int smg_lowbit_matmul_dev_noalloc(size_t m, const smg_weights *w, uint16_t *dst,
                                  const uint16_t *lhs, const ep_desc16 *ep, void *stream);
int smg_lowbit_mopa_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                        const ep_desc16 *ep, void *stream);
int smg_packed_matmul_dev(size_t m, const smg_weights *b_pack, uint16_t *dst, long dst_cs,
                          long dst_rs, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                          uint16_t beta_bits, const ep_desc16 *ep, int bf16, void *stream);

/* ---- the decode block (src/block.rs path) ----------------------------------
 * The model-level parts a Llama-style layer is built from, with the reference's
 * names and argument meaning; device pointers, asynchronous on `stream`.
 * Residual streams are f32, activations handed between parts f16, as in the
 * reference (src/linear.rs:14-29). A part's calls on one stream are ordered by
 * that stream; its scratch is the stream's own (the first call on a stream
 * allocates it, so make one before capturing a HIP graph). */
typedef struct smg_kv_cache smg_kv_cache;
typedef struct smg_attn smg_attn;
typedef struct smg_mlp smg_mlp;
typedef struct smg_block smg_block;

/* KvCache::new (src/kernels/kv_attention.rs:372-394): f16 keys and values for
 * `capacity` positions of kv_heads*head_dim values each, zeroed, score scale
 * 1/sqrt(head_dim). head_dim a multiple of 8 in 8..256, heads a positive
 * multiple of kv_heads; SMG_EINVAL otherwise. On the current device. */
int smg_kv_cache_create(size_t heads, size_t kv_heads, size_t head_dim, size_t capacity,
                        smg_kv_cache **out);
void smg_kv_cache_destroy(smg_kv_cache *c);
/* len() / capacity() / scale() (kv_attention.rs:403-453). */
int smg_kv_cache_info(const smg_kv_cache *c, size_t *len, size_t *capacity, float *scale);
/* truncate (no-op past len) / clear (len 0) (kv_attention.rs:476-484). */
int smg_kv_cache_truncate(smg_kv_cache *c, size_t len);
/* with_scale (kv_attention.rs:396-400). */
int smg_kv_cache_set_scale(smg_kv_cache *c, float scale);
/* The device storage: keys and values, capacity rows of kv_heads*head_dim f16;
 * keys() / values() (kv_attention.rs:522-531) are the first len rows. */
int smg_kv_cache_storage(const smg_kv_cache *c, uint16_t **keys, uint16_t **values);
/* The first len rows of the keys and / or values (either NULL) copied to
 * device buffers of len*kv_heads*head_dim f16 (keys() / values()). */
int smg_kv_cache_read_dev(const smg_kv_cache *c, uint16_t *keys, uint16_t *values, void *stream);
/* extend / push (kv_attention.rs:489-519) with rows rows of f16 keys and values
 * (device); SMG_EINVAL ("KvCache full") when they do not fit. */
int smg_kv_cache_extend_dev(smg_kv_cache *c, const uint16_t *k, const uint16_t *v, size_t rows,
                            void *stream);
/* attend (kv_attention.rs:537-552): one query row (heads*head_dim f32) against
 * every cached position into out (heads*head_dim f32); SMG_EINVAL when empty. */
int smg_kv_cache_attend_dev(const smg_kv_cache *c, const float *q, float *out, void *stream);
/* attention_kv_f16 (kv_attention.rs:29-78) on device arrays: q f32
 * [heads*head_dim], k / v f16 [len][kv_heads*head_dim], out f32. Replaces the
 * reference's attn_kv_f16 kernel (src/ffi.rs). */
int smg_attention_kv_f16_dev(const float *q, const uint16_t *k, const uint16_t *v, size_t len,
                             size_t heads, size_t kv_heads, size_t head_dim, float scale, float *out,
                             void *stream);
/* attention_kv_causal_f16 (kv_attention.rs:140-240) on device arrays: q f32
 * [rows][heads*head_dim], k / v f16 [start + rows][kv_heads*head_dim]; query
 * row i attends to keys 0 .. start + i, into out f32 [rows][heads*head_dim].
 * Below 32 rows each row is attention_kv_f16 over its prefix bit for bit (the
 * portable path's one_row per row); from 32 rows the call runs the blocked
 * arithmetic of the reference's attn_kv_causal_sme_f16 (probabilities rounded
 * to f16, sums in another order: within 1e-3 of the one-row call on the
 * reference's test data), as kv_attention.rs:198-201 dispatches. Replaces
 * attn_kv_causal_f16 / _sme_f16 (src/ffi.rs). */
int smg_attention_kv_causal_f16_dev(const float *q, const uint16_t *k, const uint16_t *v, size_t start,
                                    size_t rows, size_t heads, size_t kv_heads, size_t head_dim, float scale,
                                    float *out, void *stream);
/* KvCache::attend_causal (kv_attention.rs:560-578): `rows` query rows that are
 * the last `rows` cached positions, each attending causally; q and out f32
 * [rows][heads*head_dim]. SMG_EINVAL when fewer than rows positions are cached. */
int smg_kv_cache_attend_causal_dev(const smg_kv_cache *c, const float *q, size_t rows, float *out, void *stream);

/* nn::rms_norm (src/nn.rs:147-161): rows of dim f32 x to f16 y, weight f32
 * [dim]: x / sqrt(mean(x^2) + eps) * weight. */
int smg_rms_norm_f16_dev(const float *x, const float *weight, size_t rows, size_t dim, float eps,
                         uint16_t *y, void *stream);
/* nn::layer_norm (src/nn.rs:73-86,133-143): rows of dim f32 x to f16 y,
 * (x - mean) / sqrt(var + eps) * weight + bias (bias NULL: none); mean and
 * variance two passes in f32. */
int smg_layer_norm_f16_dev(const float *x, const float *weight, const float *bias, size_t rows, size_t dim,
                           float eps, uint16_t *y, void *stream);
/* GatedLinear's glu (src/linear.rs:804-826): m rows of 2n f16 values, gate and
 * up interleaved 32 columns at a time, to y = f16(act(gate) * up) [m][n];
 * act EP_ACT_SILU or EP_ACT_GELU (Gate::Silu / Gate::Gelu). */
int smg_glu_f16_dev(const uint16_t *both, size_t m, size_t n, uint32_t act, uint16_t *y,
                    void *stream);
/* Linear::accumulate for 4-bit weights (src/linear.rs:425-432): y (f32, m x n)
 * += f32(f16(x @ W)), x f16 m x k. */
int smg_q4_accumulate_dev(size_t m, const smg_weights *w, float *y, const uint16_t *x, void *stream);

/* SelfAttention::new (src/self_attention.rs:86-130): qkv Q4 with
 * (heads + 2 kv_heads)*head_dim outputs [q | k | v], out Q4 with heads*head_dim
 * inputs; rope_theta > 0 adds the NeoX rotary embedding that
 * examples/bonsai/model.rs:30-99 applies to q and k (base rope_theta, no
 * scaling), 0 none, as the library's SelfAttention. The attention takes over
 * both handles (as the Rust constructor moves its Linears): on success the
 * caller no longer destroys them. head_dim a multiple of 16 with RoPE. */
int smg_attn_create(smg_weights *qkv, smg_weights *out, size_t heads, size_t kv_heads,
                    size_t head_dim, double rope_theta, smg_attn **attn);
void smg_attn_destroy(smg_attn *a);
/* SelfAttention::accumulate (self_attention.rs:148-183): y (f32 m x width) +=
 * out(attention(qkv(x))) for x f16 (m x width) at the cache's next m
 * positions, which it appends; m > 1 attends causally (attend_rows,
 * self_attention.rs:192-240). SMG_EINVAL when the rows do not fit in the cache
 * or its heads differ. */
int smg_attn_accumulate_dev(smg_attn *a, const uint16_t *x, smg_kv_cache *cache, float *y, size_t m,
                            void *stream);

/* Mlp::gated(GatedLinear, down) (gated != 0: up holds 2*hidden outputs, gate
 * and up interleaved 32 columns at a time as GatedLinear stores them,
 * src/linear.rs:601-619) or Mlp::new(up, act, down) (src/mlp.rs:62-86); act
 * EP_ACT_SILU or EP_ACT_GELU. Takes over up and down on success. */
int smg_mlp_create(smg_weights *up, smg_weights *down, uint32_t act, int gated, smg_mlp **mlp);
void smg_mlp_destroy(smg_mlp *m);
/* Mlp::accumulate (src/mlp.rs:113-149): y (f32 m x n) += down(act(up(x))) for
 * x f16 m x k: the up GEMV with the activation (gated: glu) at its store, then
 * the down GEMV adding into y -- two kernels for up to 8 rows. */
int smg_mlp_accumulate_dev(smg_mlp *m, const uint16_t *x, float *y, size_t rows, void *stream);

/* Block::new(Norm::rms(norm1, eps1), attn, Norm::rms(norm2, eps2), mlp)
 * (src/block.rs:49-66; norms f32 [d], copied): takes over attn and mlp on
 * success (destroying the block destroys them). */
int smg_block_create(const float *norm1, float eps1, const float *norm2, float eps2, size_t d,
                     smg_attn *attn, smg_mlp *mlp, smg_block **block);
/* Block::new with either norm kind (src/nn.rs:164-214): layer != 0 is
 * Norm::layer(weight, bias, eps) (bias may be NULL), else Norm::rms(weight,
 * eps) (bias must be NULL). As smg_block_create otherwise. */
int smg_block_create_norms(const float *norm1, const float *bias1, float eps1, int layer1, const float *norm2,
                           const float *bias2, float eps2, int layer2, size_t d, smg_attn *attn, smg_mlp *mlp,
                           smg_block **block);
void smg_block_destroy(smg_block *b);
/* Block::accumulate (block.rs:90-106): x (f32, rows x d, device) += the
 * attention half, then += the MLP half, at the cache's next `rows` positions,
 * which it appends. rows = 1 with RMS norms (decode): six launches -- RMSNorm
 * + qkv + RoPE + cache append, attention splits, their merge, out + residual,
 * RMSNorm + gate/up + glu, down + residual. More rows (prefill): the norm pass,
 * the qkv GEMM, RoPE and the cache append, causal attention, the out GEMM and
 * its add, then the MLP half over all rows. */
int smg_block_accumulate_dev(smg_block *b, float *x, smg_kv_cache *cache, size_t rows, void *stream);

/* ---- host-slice forms of the model parts ------------------------------------
 * The reference's model parts take host slices (&[X] / &mut [f32]). Each entry
 * below is the synchronous host-memory twin of the *_dev entry of the same
 * name: the same arguments without the stream, every array in host memory,
 * staged through the calling thread's device buffer and stream. It returns
 * once its outputs are in host memory, and leaves them untouched when it
 * fails (the caches and handles it names are updated as by the device form).
 * Weight handles, caches and blocks stay on their device; the free functions
 * run on the current device. An f32 caller rounds x to f16 first, as the
 * reference's ModelFloat::as_f16 does (src/linear.rs:23-78). */
/* Linear::accumulate (src/linear.rs:425-432). */
int smg_q4_accumulate(size_t m, const smg_weights *w, float *y, const uint16_t *x);
/* SelfAttention::accumulate (src/self_attention.rs:148-183). */
int smg_attn_accumulate(smg_attn *a, const uint16_t *x, smg_kv_cache *cache, float *y, size_t m);
/* Mlp::accumulate (src/mlp.rs:113-149). */
int smg_mlp_accumulate(smg_mlp *m, const uint16_t *x, float *y, size_t rows);
/* Block::accumulate (src/block.rs:90-106): x f32 rows x d, updated in place. */
int smg_block_accumulate(smg_block *b, float *x, smg_kv_cache *cache, size_t rows);
/* KvCache::extend (kv_attention.rs:499-519). */
int smg_kv_cache_extend(smg_kv_cache *c, const uint16_t *k, const uint16_t *v, size_t rows);
/* keys() / values() (kv_attention.rs:522-531): len rows each, either NULL. */
int smg_kv_cache_read(const smg_kv_cache *c, uint16_t *keys, uint16_t *values);
/* KvCache::attend / attend_causal (kv_attention.rs:537-578). */
int smg_kv_cache_attend(const smg_kv_cache *c, const float *q, float *out);
int smg_kv_cache_attend_causal(const smg_kv_cache *c, const float *q, size_t rows, float *out);
/* attention_kv_f16 / attention_kv_causal_f16 (kv_attention.rs:29-78,140-240). */
int smg_attention_kv_f16(const float *q, const uint16_t *k, const uint16_t *v, size_t len, size_t heads,
                         size_t kv_heads, size_t head_dim, float scale, float *out);
int smg_attention_kv_causal_f16(const float *q, const uint16_t *k, const uint16_t *v, size_t start, size_t rows,
                                size_t heads, size_t kv_heads, size_t head_dim, float scale, float *out);
/* nn::rms_norm / nn::layer_norm (src/nn.rs:73-86,133-161). */
int smg_rms_norm_f16(const float *x, const float *weight, size_t rows, size_t dim, float eps, uint16_t *y);
int smg_layer_norm_f16(const float *x, const float *weight, const float *bias, size_t rows, size_t dim, float eps,
                       uint16_t *y);

/* ---- measurement probes (not part of the matmul path) ----------------------- */
/* One plain pass of 16-byte loads over `bytes` (a multiple of 16) of device
 * memory, writing nothing: the time floor that a single launch reading that
 * many bytes meets on this device. */
int smg_stream_read_dev(const void *p, size_t bytes, void *stream);
/* The same pass, then `out_bytes` (a multiple of 2) of device memory at `out`
 * written with 16-bit values, one per thread, as a GEMV writes its output:
 * the floor of a launch that reads `bytes` and stores a result. */
int smg_stream_read_store_dev(const void *p, size_t bytes, void *out, size_t out_bytes, void *stream);
/* Spins one wave `iters` times and stores out[0] = shader-clock ticks
 * (clock64) and out[1] = 100 MHz wall-clock ticks over the spin (device
 * memory, 3 words): out[0] / out[1] * 100 MHz is the shader clock then. */
int smg_clock_probe_dev(unsigned long long *out, unsigned iters, void *stream);

/* ---- runtime --------------------------------------------------------------- */
/* 1 when a gfx950 device is present and this library's kernels load on it. */
int smg_available(void);
/* Text of the last error on the calling thread ("" if none). */
const char *smg_last_error(void);
/* Rows at or below which Q4 runs the GEMV kernel (the reference's
 * Q4_GEMV_MAXR = 7 cut, csrc/gemm_f16f16_q4.h:129, moved to the GPU's own
 * crossover). */
size_t smg_q4_gemv_max_rows(void);

#ifdef __cplusplus
}
#endif
#endif /* SMEGEMM_GPU_H */
