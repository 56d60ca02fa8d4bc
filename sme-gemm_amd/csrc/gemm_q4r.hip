// Q4 prefill GEMM with the weights dequantized in registers:
// C = ep(to16(beta * A @ dequant(B))) for matmul_q4 / matmul_q4_ep and their
// bf16 forms past the GEMV's rows (src/kernels/q4/matmul.rs:37-103,:187-271),
// replacing run_q4_panels + unpack_q4_f16 (csrc/gemm_f16f16_q4.h:57-118) and
// q4_bf16_core (csrc/gemm_b16b16_q4.h:293). Serves f16 or bf16 activations,
// Q4_0 and Q4_1, blocks of 32 depths or more, K a multiple of 64 and
// row-major 16-byte-aligned A; every other case goes to gemm_kernel
// (gemm_mfma.hip). bf16 calls multiply on v_mfma_f32_16x16x32_bf16 with each
// weight formed in f32 and rounded to bf16 once, as the portable bf16 path.
//
// Tile: 128 rows x 256 columns, eight waves, two per SIMD. Waves w and w+4 (on
// one SIMD) own columns 64(w%4)..+63 for all 128 rows and split K: wave w
// multiplies the first 32 depths of every 64-depth step, wave w+4 the second,
// and their f32 partial tiles are added once at the end. Each wave holds 8 x 4
// MFMA tiles of 16 x 16 on v_mfma_f32_16x16x32_f16. Every weight of the tile
// is dequantized once, by the one wave that multiplies it, straight into MFMA
// B registers: no f16 weight tile is written to or read from LDS, which is
// what bounds a kernel that stages dequantized weights there. The weight is
// rounded once, f16_RNE(scale*code) (+min: one fused rounding), as the
// reference's dequant (src/kernels/q4/mod.rs:193-224).
//
// Everything a step needs goes global -> LDS by DMA (global_load_lds, no
// registers): the 128 x 64 activation tile (16-byte chunks swizzled: chunk c of
// row r at slot c ^ (r & 7), so fragment reads are conflict-free), the tile's
// raw Q4 chunks and its scales (and mins). A ring of five stages: step k+5's
// DMA is issued as soon as step k's stage is free (after step k's barrier),
// each step's barrier waits only for step k+2's DMA, and a wave reads step
// k+1's fragments from LDS while its step-k multiplies run.
#include <algorithm>
#include <atomic>

#include "kernels.h"
#include "tile_store.cuh"

namespace smg {

namespace {

constexpr int RBM = 128, RBN = 256, RNT = 512;  // tile rows, tile columns, threads
constexpr int A_BYTES = RBM * 64 * 2;           // activations: [128 rows][64 depths] f16
constexpr int B_BYTES = 2 * RBN * 16;           // raw Q4: [half][256 columns] 16-byte chunks
constexpr int S_BYTES = 2 * RBN * 2;            // scales (mins): [half][256 columns] f16
constexpr int STAGE_BYTES = A_BYTES + B_BYTES + 2 * S_BYTES;
constexpr int CS = RBN + 8;                     // halfs per staged output row
constexpr int SP = RBN + 4;                     // floats per staged split-K partial row
constexpr int NSTAGE = 5;                       // LDS ring depth
constexpr int PS = 4;                           // DMA instructions per lane per step
static_assert(RBM * CS * 2 <= NSTAGE * STAGE_BYTES, "store staging exceeds the ring");
static_assert(RBM * SP * 4 <= NSTAGE * STAGE_BYTES, "partial staging exceeds the ring");

struct RArgs {
    const uint16_t *lhs;
    const uint8_t *codes;
    const uint16_t *sc;
    const uint16_t *mn;
    StoreArgs st;
    float beta;
    long lhs_rs;
    uint32_t m, n, k, n_pad, block_shift;
    uint32_t nchunks, sc_rows;  // rows of the code and scale grids
    // split K (nsplit > 1): slice s of a tile writes its f32 sums to
    // part[s][row][col] (row stride part_ld floats); q4r_reduce finishes them
    float *part;
    uint32_t nsplit, part_ld;
    // q4r_reduce with resid ([m][n] f32): resid += the rounded f16 result
    // (the residual add), which is then not stored
    float *resid;
    // the compiled store's operands (EPV 2, 3: EpPick's a, b, act, alpha;
    // EPV 4: act, and nh the gated store's output width)
    const uint16_t *col_a, *col_b;
    uint32_t act;
    float act_alpha;
    uint32_t nh;
};

// LDS DMA: each lane's 16 (4) bytes from sbase + voff land at M0 + 16 (4) *
// lane; sbase is wave-uniform (scalar registers), voff the lane's 32-bit byte
// offset, so a step's addresses cost no vector instructions. The instructions
// are issued from inline asm so that the compiler neither tracks them nor adds
// waits of its own (it cannot tell which stage a DMA fills); the kernel's
// explicit vmcnt waits and barriers order them. The "memory" clobber keeps LDS
// reads from moving across an issue; s_nop covers the M0 write hazard. lds is a
// wave-uniform LDS byte address. (M0 has no other user in this kernel, so
// clobbering it is safe.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
                 "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void *sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase),
                 "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left unwaited).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// At most n (uniform) steps' DMA still in flight.
__device__ __forceinline__ void wait_vm_steps(int n) {
    if (n >= 3)
        wait_vm<3 * PS>();
    else if (n == 2)
        wait_vm<2 * PS>();
    else if (n == 1)
        wait_vm<PS>();
    else
        wait_vm<0>();
}

// Workgroup barrier that orders LDS accesses without waiting on outstanding
// DMA (a release fence would wait for all of it): the empty asm statements keep
// the compiler from moving memory accesses across it; the caller first waits
// for the DMA the next step reads.
__device__ __forceinline__ void barrier_lds() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Per-lane DMA offsets that do not change from step to step. Thread t loads
// activation chunks t and t+512, raw chunk t ([half t/256][column t%256]) and
// one dword of scales (waves 0-3) or mins (waves 4-7; scales again, unused,
// for Q4_0 so that every wave issues the same count). The halves are
// wave-uniform, and a cell's index is a row part plus a column part
// (cell_index), so each step's part of an address is a scalar base and the
// column's part a per-lane offset.
struct DmaSrc {
    uint32_t a[2];          // activation chunk byte offsets from A at depth 0
    uint32_t b;             // raw chunk byte offset of the column's cell in row 0
    uint32_t s;             // scale (min) pair byte offset of the column's cells in row 0
    uint32_t half_b, half_s;  // this wave's half of the step for raw chunks / scales
    const uint16_t *src_s;  // scales or mins
};

__device__ __forceinline__ void dma_step(const RArgs &g, const DmaSrc &d, const uint8_t *S, uint32_t ks,
                                         uint32_t wave) {
    const uint32_t base = lds_addr(S);
    // activations: chunk p = q*512 + t lands at byte 16p (row p/8, slot p%8)
    const uint16_t *a = g.lhs + (size_t)ks * 64;
#pragma unroll
    for (int q = 0; q < 2; q++) dma16(a, d.a[q], base + (q * 512 + wave * 64) * 16);
    // raw Q4: chunk (2ks + t/256, column t%256) at byte A_BYTES + 16t
    dma16(g.codes + cell_row_part(2 * ks + d.half_b, g.nchunks, g.n_pad) * 16, d.b, base + A_BYTES + wave * 64 * 16);
    // scales (mins): [half][column] f16, two per lane
    const size_t row = (size_t)(((2 * ks + d.half_s) * 32) >> g.block_shift);
    dma4(d.src_s + cell_row_part(row, g.sc_rows, g.n_pad), d.s, base + A_BYTES + B_BYTES + wave * 256);
}

// One 32-depth half of a step as LDS reads: 8 activation fragments and, per
// column tile, the raw dword and scale (min) of this lane's 8 depths.
// (32-bit vector types, not arrays of 16-bit values: the fields stay in
// registers, one element per register)
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
struct Half {
    u32x4_t a[8];
    u32x4_t q, s, mn;
};

// This lane's LDS byte offsets within a stage (constant over the loop).
struct ReadOff {
    uint32_t a, q, s;  // first activation fragment, first raw dword, first scale
};

__device__ __forceinline__ ReadOff read_offsets(int kk, int cw, int lane) {
    const int lr = lane % 16, lg = lane / 16;
    ReadOff o;
    o.a = lr * 128 + (((kk * 4 + lg) ^ (lr & 7)) << 4);  // row & 7 == lr & 7 for rows 16i + lr
    o.q = A_BYTES + (kk * 256 + cw * 64 + lr) * 16 + lg * 4;
    o.s = A_BYTES + B_BYTES + kk * 512 + (cw * 64 + lr) * 2;
    return o;
}

typedef const __attribute__((address_space(3))) uint8_t lds_u8_t;
template <class T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
    return *(const __attribute__((address_space(3))) T *)(lds_u8_t *)(uintptr_t)addr;
}

// Stage at LDS byte address sb: row tile i's fragment at o.a + 2048 i, column
// tile jt's raw dword at o.q + 256 jt and scale at o.s + 32 jt (min S_BYTES
// further on).
template <bool AFFINE>
__device__ __forceinline__ void read_half(uint32_t sb, const ReadOff &o, Half &h) {
#pragma unroll
    for (int i = 0; i < 8; i++) h.a[i] = lds_load<u32x4_t>(sb + o.a + 2048 * i);
#pragma unroll
    for (int jt = 0; jt < 4; jt++) {
        h.q[jt] = lds_load<uint32_t>(sb + o.q + 256 * jt);
        h.s[jt] = lds_load<uint16_t>(sb + o.s + 32 * jt);
        if (AFFINE) h.mn[jt] = lds_load<uint16_t>(sb + o.s + S_BYTES + 32 * jt);
    }
}

// One column tile's 8 MFMAs (row tiles i = 0..7, B operand b) with the next
// column tile's dequant interleaved, in a fixed order: two vector instructions
// between MFMAs keep the matrix core fed (the compiler's own schedule clusters
// them). The dequant is q4_deq8 / q4_deq8_affine: v_bfi_b32 puts each biased
// nibble under an f16 exponent (magic 0x6400 | u = 1024 + u; 0x5400 | u << 4 =
// 64 + u), a packed add of -1032 / -72 leaves the exact code, then one packed
// multiply by the scale pair s2 (Q4_0) or one packed fma with the min pair m2
// (Q4_1) rounds the weight once. nb must not be read by an MFMA for two wait
// states after its last write: each group ends with s_nop 1. nb was last read
// by the MFMAs three groups earlier (four rotating buffers).
template <bool AFFINE>
__device__ __forceinline__ void mma8_deq(float4_t &c0, float4_t &c1, float4_t &c2, float4_t &c3, float4_t &c4,
                                         float4_t &c5, float4_t &c6, float4_t &c7, const u32x4_t (&a)[8],
                                         const u32x4_t &b, u32x4_t &nb, uint32_t q, uint32_t s2, uint32_t m2,
                                         uint32_t mag_lo, uint32_t mag_hi) {
    uint32_t t;
    if (AFFINE) {
        asm volatile(
            "v_mfma_f32_16x16x32_f16 %[c0], %[a0], %[b], %[c0]\n\t"
            "v_lshrrev_b32 %[t], 8, %[q]\n\t"
            "v_bfi_b32 %[n0], %[m1], %[q], %[ml]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c1], %[a1], %[b], %[c1]\n\t"
            "v_bfi_b32 %[n1], %[m2m], %[q], %[mh]\n\t"
            "v_bfi_b32 %[n2], %[m1], %[t], %[ml]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c2], %[a2], %[b], %[c2]\n\t"
            "v_bfi_b32 %[n3], %[m2m], %[t], %[mh]\n\t"
            "v_pk_add_f16 %[n0], %[n0], %[ol]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c3], %[a3], %[b], %[c3]\n\t"
            "v_pk_add_f16 %[n1], %[n1], %[oh]\n\t"
            "v_pk_add_f16 %[n2], %[n2], %[ol]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c4], %[a4], %[b], %[c4]\n\t"
            "v_pk_add_f16 %[n3], %[n3], %[oh]\n\t"
            "v_pk_fma_f16 %[n0], %[n0], %[s2], %[mn]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c5], %[a5], %[b], %[c5]\n\t"
            "v_pk_fma_f16 %[n1], %[n1], %[s2], %[mn]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c6], %[a6], %[b], %[c6]\n\t"
            "v_pk_fma_f16 %[n2], %[n2], %[s2], %[mn]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c7], %[a7], %[b], %[c7]\n\t"
            "v_pk_fma_f16 %[n3], %[n3], %[s2], %[mn]\n\t"
            "s_nop 1"
            : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [c3] "+v"(c3), [c4] "+v"(c4), [c5] "+v"(c5),
              [c6] "+v"(c6), [c7] "+v"(c7), [n0] "=&v"(nb.x), [n1] "=&v"(nb.y), [n2] "=&v"(nb.z),
              [n3] "=&v"(nb.w), [t] "=&v"(t)
            : [a0] "v"(a[0]), [a1] "v"(a[1]), [a2] "v"(a[2]), [a3] "v"(a[3]), [a4] "v"(a[4]), [a5] "v"(a[5]),
              [a6] "v"(a[6]), [a7] "v"(a[7]), [b] "v"(b), [q] "v"(q), [s2] "v"(s2), [mn] "v"(m2),
              [ml] "v"(mag_lo), [mh] "v"(mag_hi), [m1] "s"(0x000F000Fu), [m2m] "s"(0x00F000F0u),
              [ol] "s"(0xE408E408u), [oh] "s"(0xD480D480u));
    } else {
        (void)m2;
        asm volatile(
            "v_mfma_f32_16x16x32_f16 %[c0], %[a0], %[b], %[c0]\n\t"
            "v_lshrrev_b32 %[t], 8, %[q]\n\t"
            "v_bfi_b32 %[n0], %[m1], %[q], %[ml]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c1], %[a1], %[b], %[c1]\n\t"
            "v_bfi_b32 %[n1], %[m2m], %[q], %[mh]\n\t"
            "v_bfi_b32 %[n2], %[m1], %[t], %[ml]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c2], %[a2], %[b], %[c2]\n\t"
            "v_bfi_b32 %[n3], %[m2m], %[t], %[mh]\n\t"
            "v_pk_add_f16 %[n0], %[n0], %[ol]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c3], %[a3], %[b], %[c3]\n\t"
            "v_pk_add_f16 %[n1], %[n1], %[oh]\n\t"
            "v_pk_add_f16 %[n2], %[n2], %[ol]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c4], %[a4], %[b], %[c4]\n\t"
            "v_pk_add_f16 %[n3], %[n3], %[oh]\n\t"
            "v_pk_mul_f16 %[n0], %[n0], %[s2]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c5], %[a5], %[b], %[c5]\n\t"
            "v_pk_mul_f16 %[n1], %[n1], %[s2]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c6], %[a6], %[b], %[c6]\n\t"
            "v_pk_mul_f16 %[n2], %[n2], %[s2]\n\t"
            "v_mfma_f32_16x16x32_f16 %[c7], %[a7], %[b], %[c7]\n\t"
            "v_pk_mul_f16 %[n3], %[n3], %[s2]\n\t"
            "s_nop 1"
            : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [c3] "+v"(c3), [c4] "+v"(c4), [c5] "+v"(c5),
              [c6] "+v"(c6), [c7] "+v"(c7), [n0] "=&v"(nb.x), [n1] "=&v"(nb.y), [n2] "=&v"(nb.z),
              [n3] "=&v"(nb.w), [t] "=&v"(t)
            : [a0] "v"(a[0]), [a1] "v"(a[1]), [a2] "v"(a[2]), [a3] "v"(a[3]), [a4] "v"(a[4]), [a5] "v"(a[5]),
              [a6] "v"(a[6]), [a7] "v"(a[7]), [b] "v"(b), [q] "v"(q), [s2] "v"(s2), [ml] "v"(mag_lo),
              [mh] "v"(mag_hi), [m1] "s"(0x000F000Fu), [m2m] "s"(0x00F000F0u), [ol] "s"(0xE408E408u),
              [oh] "s"(0xD480D480u));
    }
}

// The bf16 form of mma8_deq (matmul_q4_bf16 prefill): v_mfma_f32_16x16x32_bf16
// with the weights formed as q4_deq8_bf16 forms them -- the biased nibble
// under an f16 exponent less its offset is the exact code as f16, then
// v_fma_mix_f32 gives f32(code) * f32(scale) + f32(min) (min -0 for Q4_0: the
// product unchanged) with the f32 rounding of the reference's f32 dequant, and
// v_cvt_pk_bf16_f32 rounds each pair to bf16 once (src/kernels/q4/mod.rs
// dequant to bf16). s1 holds the f16 scale in its low half, mf the min as f32.
__device__ __forceinline__ void mma8_deq_bf16(float4_t &c0, float4_t &c1, float4_t &c2, float4_t &c3, float4_t &c4,
                                              float4_t &c5, float4_t &c6, float4_t &c7, const u32x4_t (&a)[8],
                                              const u32x4_t &b, u32x4_t &nb, uint32_t q, uint32_t s1, float mf,
                                              uint32_t mag_lo, uint32_t mag_hi) {
    uint32_t t;
    float f0, f1;
    asm volatile(
        "v_mfma_f32_16x16x32_bf16 %[c0], %[a0], %[b], %[c0]\n\t"
        "v_lshrrev_b32 %[t], 8, %[q]\n\t"
        "v_bfi_b32 %[n0], %[m1], %[q], %[ml]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c1], %[a1], %[b], %[c1]\n\t"
        "v_bfi_b32 %[n1], %[m2m], %[q], %[mh]\n\t"
        "v_bfi_b32 %[n2], %[m1], %[t], %[ml]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c2], %[a2], %[b], %[c2]\n\t"
        "v_bfi_b32 %[n3], %[m2m], %[t], %[mh]\n\t"
        "v_pk_add_f16 %[n0], %[n0], %[ol]\n\t"
        "v_pk_add_f16 %[n1], %[n1], %[oh]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c3], %[a3], %[b], %[c3]\n\t"
        "v_pk_add_f16 %[n2], %[n2], %[ol]\n\t"
        "v_pk_add_f16 %[n3], %[n3], %[oh]\n\t"
        "v_fma_mix_f32 %[f0], %[n0], %[s1], %[mf] op_sel_hi:[1,1,0]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c4], %[a4], %[b], %[c4]\n\t"
        "v_fma_mix_f32 %[f1], %[n0], %[s1], %[mf] op_sel:[1,0,0] op_sel_hi:[1,1,0]\n\t"
        "v_cvt_pk_bf16_f32 %[n0], %[f0], %[f1]\n\t"
        "v_fma_mix_f32 %[f0], %[n1], %[s1], %[mf] op_sel_hi:[1,1,0]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c5], %[a5], %[b], %[c5]\n\t"
        "v_fma_mix_f32 %[f1], %[n1], %[s1], %[mf] op_sel:[1,0,0] op_sel_hi:[1,1,0]\n\t"
        "v_cvt_pk_bf16_f32 %[n1], %[f0], %[f1]\n\t"
        "v_fma_mix_f32 %[f0], %[n2], %[s1], %[mf] op_sel_hi:[1,1,0]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c6], %[a6], %[b], %[c6]\n\t"
        "v_fma_mix_f32 %[f1], %[n2], %[s1], %[mf] op_sel:[1,0,0] op_sel_hi:[1,1,0]\n\t"
        "v_cvt_pk_bf16_f32 %[n2], %[f0], %[f1]\n\t"
        "v_fma_mix_f32 %[f0], %[n3], %[s1], %[mf] op_sel_hi:[1,1,0]\n\t"
        "v_mfma_f32_16x16x32_bf16 %[c7], %[a7], %[b], %[c7]\n\t"
        "v_fma_mix_f32 %[f1], %[n3], %[s1], %[mf] op_sel:[1,0,0] op_sel_hi:[1,1,0]\n\t"
        "v_cvt_pk_bf16_f32 %[n3], %[f0], %[f1]\n\t"
        "s_nop 1"
        : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [c3] "+v"(c3), [c4] "+v"(c4), [c5] "+v"(c5),
          [c6] "+v"(c6), [c7] "+v"(c7), [n0] "=&v"(nb.x), [n1] "=&v"(nb.y), [n2] "=&v"(nb.z),
          [n3] "=&v"(nb.w), [t] "=&v"(t), [f0] "=&v"(f0), [f1] "=&v"(f1)
        : [a0] "v"(a[0]), [a1] "v"(a[1]), [a2] "v"(a[2]), [a3] "v"(a[3]), [a4] "v"(a[4]), [a5] "v"(a[5]),
          [a6] "v"(a[6]), [a7] "v"(a[7]), [b] "v"(b), [q] "v"(q), [s1] "v"(s1), [mf] "v"(mf),
          [ml] "v"(mag_lo), [mh] "v"(mag_hi), [m1] "s"(0x000F000Fu), [m2m] "s"(0x00F000F0u),
          [ol] "s"(0xE408E408u), [oh] "s"(0xD480D480u));
}

template <int N>
struct IntC {
    static constexpr int value = N;
};

__device__ __forceinline__ uint32_t pair16(uint32_t h) { return (h & 0xFFFFu) | (h << 16); }

// The first column tile's B operand of a step (plain code, before the groups).
template <bool AFFINE, bool BF16>
__device__ __forceinline__ u32x4_t deq_first(const Half &h, uint32_t mag_lo, uint32_t mag_hi) {
    const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)h.s[0]);
    const half2_t s2 = {s, s};
    uint4 b;
    if (BF16) {
        b = q4_deq8_bf16(h.q[0], h.s[0], AFFINE ? f16_to_f32((uint16_t)h.mn[0]) : -0.0f, mag_lo, mag_hi);
    } else if (AFFINE) {
        const _Float16 mv = __builtin_bit_cast(_Float16, (uint16_t)h.mn[0]);
        b = q4_deq8_affine(h.q[0], s2, (half2_t){mv, mv}, mag_lo, mag_hi);
    } else {
        b = q4_deq8(h.q[0], s2, mag_lo, mag_hi);
    }
    return (u32x4_t){b.x, b.y, b.z, b.w};
}

// A step's 32 MFMAs: column tile jt multiplies B operand bb[jt] (dequantized
// during the previous group) and dequantizes bb[jt+1] -- for the last tile,
// the next step's first (raw operands in nxt).
template <bool AFFINE, bool BF16>
__device__ __forceinline__ void mma_step(const Half &cur, const Half &nxt, float4_t (&acc)[8][4],
                                         u32x4_t (&bb)[4], uint32_t mag_lo, uint32_t mag_hi) {
#pragma unroll
    for (int jt = 0; jt < 4; jt++) {
        const Half &src = jt < 3 ? cur : nxt;
        const int nj = (jt + 1) % 4;
        if constexpr (BF16)
            mma8_deq_bf16(acc[0][jt], acc[1][jt], acc[2][jt], acc[3][jt], acc[4][jt], acc[5][jt], acc[6][jt],
                          acc[7][jt], cur.a, bb[jt], bb[nj], src.q[nj], src.s[nj],
                          AFFINE ? f16_to_f32((uint16_t)src.mn[nj]) : -0.0f, mag_lo, mag_hi);
        else
            mma8_deq<AFFINE>(acc[0][jt], acc[1][jt], acc[2][jt], acc[3][jt], acc[4][jt], acc[5][jt], acc[6][jt],
                             acc[7][jt], cur.a, bb[jt], bb[nj], src.q[nj], pair16(src.s[nj]),
                             AFFINE ? pair16(src.mn[nj]) : 0u, mag_lo, mag_hi);
    }
}

// EPV: the store's op-graph, compiled for the common shapes (pick_ep): 0 any
// graph (the interpreted store), 1 none, 2 [add_col] + act, 3 [mul_col,
// add_col] + act; 4 the gated store (ep_store_glu8, f16). SPLIT kernels store
// partials only (EPV 0).
template <bool AFFINE, bool SPLIT, int EPV = 0, bool BF16 = false>
__global__ void __launch_bounds__(RNT) gemm_q4r(RArgs g, EpArgs ep) {
    static_assert(!SPLIT || EPV == 0, "a split kernel's store is q4r_reduce's");
    static_assert(EPV != 4 || !BF16, "the gated store is f16");
    __shared__ __align__(16) uint8_t ring[NSTAGE * STAGE_BYTES];
    __shared__ __align__(16) float epv[EPV == 0 ? EP_FUSED * (RBN + RBM) : 4];

    const uint32_t mtiles = (g.m + RBM - 1) / RBM;
    const int t = threadIdx.x, lane = t % 64;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);  // uniform: DMA bases, branches
    const int cw = wave % 4, kh = wave / 4;  // column block, half of each step
    // this workgroup's tile and its steps: all of K, or (SPLIT) slice `slice`
    // of nsplit, the tile index running fastest so that consecutive
    // workgroups still share a weight slice
    uint32_t tile = xcd_tile(blockIdx.x, gridDim.x), slice = 0, ks0 = 0, ksteps = g.k / 64;  // >= 1
    if constexpr (SPLIT) {
        const uint32_t tiles = gridDim.x / g.nsplit;
        slice = tile / tiles;
        tile %= tiles;
        ks0 = slice * ksteps / g.nsplit;  // nsplit <= ksteps: every slice has a step
        ksteps = (slice + 1) * ksteps / g.nsplit - ks0;
    }

    // the bfi magics live in VGPRs (a VOP3 takes one scalar operand)
    uint32_t mag_lo = 0x64006400u, mag_hi = 0x54005400u;
    asm volatile("" : "+v"(mag_lo), "+v"(mag_hi));
    const uint32_t ring0 = lds_addr(ring);
    const ReadOff ro = read_offsets(kh, cw, lane);

    // The tile's K loop, the pair's sum and the store. (Written as a lambda
    // that the kernel calls once: in this form the compiler keeps the
    // per-lane read offsets as immediates of paired ds_read2st64 reads instead
    // of adding a base register per read.)
    auto run_tile = [&](uint32_t tile) __attribute__((always_inline)) {
        // column-tile-major order
        const uint32_t tm = tile % mtiles, tn = tile / mtiles;
        const uint32_t row0 = tm * RBM, col0 = tn * RBN;

        // Rows past m and columns past n_pad read clamped (valid) addresses;
        // their results are never stored.
        DmaSrc d;
        {
            const uint32_t c = (t % 8) ^ ((t / 8) % 8);  // source chunk of slot t%8 in row t/8 (+64q)
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const uint32_t row = min(row0 + q * 64 + t / 8, g.m - 1);
                d.a[q] = (uint32_t)(((size_t)row * g.lhs_rs + c * 8) * 2);
            }
            const uint32_t cb = min(col0 + t % 256, g.n_pad - 1);
            const uint32_t cs = min(col0 + 2 * (t % 128), g.n_pad - 2);  // even: cs, cs+1 share a tile
            d.b = (uint32_t)cell_col_part(cb, g.nchunks, g.n_pad) * 16;
            d.s = (uint32_t)cell_col_part(cs, g.sc_rows, g.n_pad) * 2;
            d.half_b = wave / 4;
            d.half_s = (wave % 4) / 2;
            d.src_s = (AFFINE && wave >= 4) ? g.mn : g.sc;
        }
        const uint32_t last = ksteps - 1;

        float4_t acc[8][4];
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int jt = 0; jt < 4; jt++) acc[i][jt] = (float4_t){0.f, 0.f, 0.f, 0.f};

        if constexpr (SPLIT) {
            // a slice of a few steps issues no loads past its last step, so
            // nothing is left in flight to drain at its end
#pragma unroll
            for (int j = 0; j < NSTAGE; j++)
                if ((uint32_t)j <= last) dma_step(g, d, ring + j * STAGE_BYTES, ks0 + j, wave);
            wait_vm_steps(min((int)last, NSTAGE - 1) - 1);  // steps 0 and 1 landed
        } else {
#pragma unroll
            for (int j = 0; j < NSTAGE; j++) dma_step(g, d, ring + j * STAGE_BYTES, min((uint32_t)j, last), wave);
            wait_vm<(NSTAGE - 2) * PS>();  // steps 0 and 1 landed
        }
        barrier_lds();

        // Step ks: step ks+1's fragments are read (its stage was published by
        // the barrier ending step ks-1) while step ks multiplies; then step
        // ks+2's DMA is waited for and the barrier publishes it -- and frees
        // stage ks%5, whose fragments every wave has multiplied -- and step
        // ks+5's DMA is issued into that stage. Steps past the end re-load the
        // last step into a free stage (SPLIT: issue nothing) and read a stage
        // nobody multiplies.
        u32x4_t bb[4];  // B operands of the four column tiles, rotating
        auto step = [&](uint32_t ks, const Half &cur, Half &nxt) {
            uint32_t sb = ring0 + ((ks + 1) % NSTAGE) * STAGE_BYTES;
            asm volatile("" : "+s"(sb));  // opaque: one base add per operand kind, constant offsets after
            read_half<AFFINE>(sb, ro, nxt);
            mma_step<AFFINE, BF16>(cur, nxt, acc, bb, mag_lo, mag_hi);
            if constexpr (SPLIT) {
                // issued: steps up to min(ks + 4, last); step ks+2 must land
                const int after = (int)last - (int)ks - 2;
                wait_vm_steps(after > 2 ? 2 : after);
                barrier_lds();
                if (ks + NSTAGE <= last) dma_step(g, d, ring + (ks % NSTAGE) * STAGE_BYTES, ks0 + ks + NSTAGE, wave);
            } else {
                wait_vm<(NSTAGE - 3) * PS>();
                barrier_lds();
                dma_step(g, d, ring + (ks % NSTAGE) * STAGE_BYTES, min(ks + NSTAGE, last), wave);
            }
        };
        Half h0, h1;
        read_half<AFFINE>(ring0, ro, h0);
        bb[0] = deq_first<AFFINE, BF16>(h0, mag_lo, mag_hi);
        uint32_t ks = 0;
        for (; ks + 2 <= ksteps; ks += 2) {
            step(ks, h0, h1);
            step(ks + 1, h1, h0);
        }
        if (ks < ksteps) step(ks, h0, h1);
        wait_vm<0>();
        __syncthreads();

        float *colv = epv, *rowv = epv + EP_FUSED * RBN;
        // the op-graph's vectors first: their global loads overlap the exchange
        if constexpr (!SPLIT && EPV == 0) ep_load_vectors<BF16, RBM, RBN, RNT>(g.st, ep, colv, rowv, row0, col0);
        EpCols cv;
        if constexpr (EPV == 2 || EPV == 3) ep_cols_load<EPV>(g.col_a, g.col_b, col0 + (t % (RBN / 8)) * 8, g.n, cv);

        // The pair's partial tiles: each wave hands the other the half of its
        // f32 tile that the other finishes (wave w keeps row tiles 0-3, wave
        // w+4 row tiles 4-7) through LDS, 16 bytes per lane and
        // lane-contiguous (conflict-free). f32 addition commutes, so either
        // wave's sum is the same value. Then each wave rounds beta * sum to f16
        // into the staged tile ([128][CS]; a lane holds
        // D[4*(lane/16)+v][lane%16] of each 16x16 tile) -- or (SPLIT) stages
        // the f32 sums ([128][SP]) for all eight waves to write the rows below
        // m and the columns below part_ld to the slice's part of the partial
        // buffer, 16 bytes a lane.
        uint16_t *stg = (uint16_t *)ring;
        auto finish_half = [&](auto keep_c) {
            constexpr int KEEP = decltype(keep_c)::value, GIVE = 4 - KEEP;
            float4_t *mine = (float4_t *)ring + wave * 1024;  // 16 KB per wave
            const float4_t *other = (const float4_t *)ring + ((wave + 4) % 8) * 1024;
            // SPLIT, the tile's rows all below 64: row tiles 4-7 are padding,
            // neither handed over nor finished
            const bool pad_hi = SPLIT && row0 + 64 >= g.m;
            if (!(pad_hi && GIVE == 4)) {
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int jt = 0; jt < 4; jt++) mine[(i * 4 + jt) * 64 + lane] = acc[GIVE + i][jt];
            }
            __syncthreads();
            if (pad_hi && KEEP == 4) {
                __syncthreads();  // the SPLIT branch's barrier
                return;
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jt = 0; jt < 4; jt++) acc[KEEP + i][jt] += other[(i * 4 + jt) * 64 + lane];
            const int lr = lane % 16, lg = lane / 16;
            if constexpr (SPLIT) {
                __syncthreads();  // the staged tile overwrites the exchange
                float *sf = (float *)ring;
#pragma unroll
                for (int i = KEEP; i < KEEP + 4; i++)
#pragma unroll
                    for (int jt = 0; jt < 4; jt++)
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            sf[(i * 16 + lg * 4 + v) * SP + cw * 64 + jt * 16 + lr] = acc[i][jt][v];
                return;
            }
            __syncthreads();  // the staged tile overwrites the exchange
#pragma unroll
            for (int i = KEEP; i < KEEP + 4; i++)
#pragma unroll
                for (int jt = 0; jt < 4; jt++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        stg[(i * 16 + lg * 4 + v) * CS + cw * 64 + jt * 16 + lr] =
                            from_f32<BF16>(0.0f + g.beta * acc[i][jt][v]);
        };
        static_assert(8 * 1024 * sizeof(float4_t) <= NSTAGE * STAGE_BYTES, "exchange exceeds the ring");
        if (kh == 0)
            finish_half(IntC<0>{});
        else
            finish_half(IntC<4>{});
        __syncthreads();
        if constexpr (SPLIT) {
            // thread t: float4 t % 64 of rows t / 64 + 8 j, below m and part_ld
            const float *sf = (const float *)ring;
            const uint32_t c4 = (t % 64) * 4;
            if (col0 + c4 >= g.part_ld) return;
            float *pp = g.part + ((size_t)slice * g.m + row0) * g.part_ld + col0 + c4;
#pragma unroll
            for (int j = 0; j < RBM / 8; j++) {
                const int r = t / 64 + 8 * j;
                if (row0 + r >= g.m) break;
                *(float4_t *)(pp + (size_t)r * g.part_ld) = *(const float4_t *)(sf + r * SP + c4);
            }
            return;
        }
        // Store: groups of 8 columns through the op-graph by all eight waves.
        // thread t: column group t % 32, rows t / 32 + 16 j
        static_assert(RNT % (RBN / 8) == 0, "each thread keeps one column group");
        if constexpr (EPV == 0)
            ep_store_rows<BF16, RBM, RBN, RBM * (RBN / 8) / RNT>(g.st, ep, colv, rowv, stg, CS, t / (RBN / 8),
                                                                 RNT / (RBN / 8), (t % (RBN / 8)) * 8, row0, col0);
        else if constexpr (EPV == 4)  // thread t: gate group t % 16, rows t / 16 + 32 j
            ep_store_glu8<RBM * (RBN / 16) / RNT>(g.st, g.act, g.nh, stg, CS, t / (RBN / 16), RNT / (RBN / 16),
                                                  (t % (RBN / 16)) * 16, row0, col0);
        else
            ep_store_rows_c<BF16, RBM * (RBN / 8) / RNT, EPV>(g.st, g.act, g.act_alpha, cv, stg, CS, t / (RBN / 8),
                                                              RNT / (RBN / 8), (t % (RBN / 8)) * 8, row0, col0);
    };
    run_tile(tile);  // consecutive workgroups share a weight tile
}

// Split K's second pass: C = ep(to16(beta * sum over the slices of part)),
// the slices added in order (the result does not depend on which workgroup
// finished first). Tile: QR_BM rows x 256 columns, one thread per row and
// column group of 8 (two 16-byte loads a slice, four slices' loads issued
// together), stored through the op-graph as the GEMM's own store does. The
// tile is short so that even a few rows make a grid of many workgroups: the
// pass is bound by how many loads are in flight.
constexpr int QR_BN = 256, QR_NT = 256, QR_BM = QR_NT / (QR_BN / 8);
template <bool BF16>
__global__ void __launch_bounds__(QR_NT) q4r_reduce(RArgs g, EpArgs ep) {
    __shared__ __align__(16) float epv[EP_FUSED * (QR_BN + QR_BM)];
    const uint32_t mtiles = (g.m + QR_BM - 1) / QR_BM;
    const uint32_t tile = xcd_tile(blockIdx.x, gridDim.x);
    const uint32_t row0 = (tile % mtiles) * QR_BM, col0 = (tile / mtiles) * QR_BN;
    float *colv = epv, *rowv = epv + EP_FUSED * QR_BN;
    ep_load_vectors<BF16, QR_BM, QR_BN, QR_NT>(g.st, ep, colv, rowv, row0, col0);
    __syncthreads();
    const int t = threadIdx.x;
    const uint32_t cl = (t % (QR_BN / 8)) * 8, rl = t / (QR_BN / 8);
    if (col0 + cl >= g.n || row0 + rl >= g.m) return;  // no barrier follows
    const size_t stride = (size_t)g.m * g.part_ld / 4;  // float4s per slice
    const float4_t *p = (const float4_t *)(g.part + (size_t)(row0 + rl) * g.part_ld + col0 + cl);
    float4_t s0 = p[0], s1 = p[1];
    uint32_t sl = 1;
    for (; sl + 4 <= g.nsplit; sl += 4) {
        float4_t v[4][2];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            v[u][0] = p[(sl + u) * stride];
            v[u][1] = p[(sl + u) * stride + 1];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            s0 += v[u][0];
            s1 += v[u][1];
        }
    }
    for (; sl < g.nsplit; sl++) {
        s0 += p[sl * stride];
        s1 += p[sl * stride + 1];
    }
    uint32_t w4[4];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        w4[e] = (uint32_t)from_f32<BF16>(0.0f + g.beta * s0[2 * e]) |
                ((uint32_t)from_f32<BF16>(0.0f + g.beta * s0[2 * e + 1]) << 16);
        w4[2 + e] = (uint32_t)from_f32<BF16>(0.0f + g.beta * s1[2 * e]) |
                    ((uint32_t)from_f32<BF16>(0.0f + g.beta * s1[2 * e + 1]) << 16);
    }
    if (g.resid) {  // f16 only (launch_q4r_resid)
        const uint32_t row = row0 + rl, col = col0 + cl, ne = g.n - col < 8 ? g.n - col : 8;
        float *yp = g.resid + (size_t)row * g.n + col;
        if (ne == 8 && ((uintptr_t)yp & 15) == 0) {
            float4_t y0 = *(const float4_t *)yp, y1 = *(const float4_t *)(yp + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                y0[e] = y0[e] + f16_to_f32((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
                y1[e] = y1[e] + f16_to_f32((uint16_t)(w4[2 + e / 2] >> (16 * (e % 2))));
            }
            *(float4_t *)yp = y0;
            *(float4_t *)(yp + 4) = y1;
            return;
        }
        for (uint32_t e = 0; e < ne; e++) yp[e] = yp[e] + f16_to_f32((uint16_t)(w4[e / 2] >> (16 * (e % 2))));
        return;
    }
    ep_store8<BF16, QR_BM, QR_BN>(g.st, ep, colv, rowv, make_uint4(w4[0], w4[1], w4[2], w4[3]), rl, cl, row0,
                                   col0);
}

}  // namespace

bool q4r_supported(const WDev &w, size_t m, long lhs_cs, long lhs_rs, const uint16_t *lhs, bool bf16) {
    (void)bf16;  // f16 and bf16 activations alike
    return w.kind == W_Q4 && m > 0 && w.k >= 64 && w.k % 64 == 0 && w.block >= 32 &&
           lhs_cs == 1 && lhs_rs % 8 == 0 && lhs_rs >= (long)w.k && ((uintptr_t)lhs & 15) == 0 &&
           m * (size_t)lhs_rs * 2 < ((size_t)1 << 31) &&  // 32-bit DMA offsets
           cell_grid_rows(w.nchunks) * w.n_pad * 16 < ((size_t)1 << 32);
}

int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cus[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// One 512-thread workgroup of gemm_q4r fills a compute unit's LDS. A grid of
// fewer tiles than half the compute units leaves most of them idle for the
// whole of K (at K = 4096, 33 to 256 rows take about 52 us at N = 4096 with 16
// to 32 tiles): then K is cut into as many slices as fill the compute units
// once, each at least Q4R_MIN_SLICE_STEPS steps of 64 depths, and at most
// Q4R_MAX_SPLIT slices: every slice adds m x N f32 partials that the end of
// the kernel writes back from L2 and the reduction reads again (16 slices
// measured 1-2 us slower than 8 at N = 4096, K = 4096).
constexpr uint32_t Q4R_MIN_SLICE_STEPS = 2, Q4R_MAX_SPLIT = 8;
uint32_t q4r_nsplit(const WDev &w, size_t m) {
    if (w.kind != W_Q4 || w.k < 64 || w.k % 64 != 0 || w.block < 32) return 1;  // not gemm_q4r's
    const size_t tiles = ((m + RBM - 1) / RBM) * ((w.n + RBN - 1) / RBN);
    const size_t cus = (size_t)device_cus();
    if (tiles == 0 || tiles * 2 > cus) return 1;
    const size_t by_k = std::max<size_t>(1, (w.k / 64) / Q4R_MIN_SLICE_STEPS);
    return (uint32_t)std::min(std::min(cus / tiles, by_k), (size_t)Q4R_MAX_SPLIT);
}

size_t q4r_split_bytes(const WDev &w, size_t m) {
    const uint32_t ns = q4r_nsplit(w, m);
    return ns > 1 ? (size_t)ns * m * ((w.n + 7) / 8 * 8) * sizeof(float) : 0;
}

static RArgs q4r_args(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs, const uint16_t *lhs,
                      long lhs_rs, float beta) {
    RArgs g = {};
    g.lhs = lhs;
    g.codes = w.codes;
    g.sc = w.scales;
    g.mn = w.mins;
    g.st = {dst, dst_rs, dst_cs, (uint32_t)m, (uint32_t)w.n, 0.0f, 0u};
    g.beta = beta;
    g.lhs_rs = lhs_rs;
    g.m = (uint32_t)m;
    g.n = (uint32_t)w.n;
    g.k = (uint32_t)w.k;
    g.n_pad = (uint32_t)w.n_pad;
    g.block_shift = (uint32_t)__builtin_ctzll(w.block);
    g.nchunks = (uint32_t)w.nchunks;
    g.sc_rows = (uint32_t)w.sc_rows;
    return g;
}

hipError_t launch_q4r(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                      const uint16_t *lhs, long lhs_rs, float beta, const EpArgs &ep, float *part,
                      size_t part_bytes, bool bf16, hipStream_t s) {
    RArgs g = q4r_args(w, m, dst, dst_cs, dst_rs, lhs, lhs_rs, beta);
    const uint32_t tiles = (uint32_t)(((m + RBM - 1) / RBM) * ((w.n + RBN - 1) / RBN));
    const size_t slice_bytes = m * ((w.n + 7) / 8 * 8) * sizeof(float);
    const uint32_t ns = part ? (uint32_t)std::min<size_t>(q4r_nsplit(w, m), part_bytes / slice_bytes) : 1;
    if (ns <= 1) {
        const EpPick pk = pick_ep(ep);
        g.col_a = pk.a;
        g.col_b = pk.b;
        g.act = pk.act;
        g.act_alpha = pk.alpha;
#define SMG_Q4R_LAUNCH(AF, BF)                                                                              \
    switch (pk.v) {                                                                                         \
    case 1: hipLaunchKernelGGL((gemm_q4r<AF, false, 1, BF>), dim3(tiles), dim3(RNT), 0, s, g, ep); break; \
    case 2: hipLaunchKernelGGL((gemm_q4r<AF, false, 2, BF>), dim3(tiles), dim3(RNT), 0, s, g, ep); break; \
    case 3: hipLaunchKernelGGL((gemm_q4r<AF, false, 3, BF>), dim3(tiles), dim3(RNT), 0, s, g, ep); break; \
    default: hipLaunchKernelGGL((gemm_q4r<AF, false, 0, BF>), dim3(tiles), dim3(RNT), 0, s, g, ep); break; \
    }
        if (w.mins && bf16) {
            SMG_Q4R_LAUNCH(true, true)
        } else if (w.mins) {
            SMG_Q4R_LAUNCH(true, false)
        } else if (bf16) {
            SMG_Q4R_LAUNCH(false, true)
        } else {
            SMG_Q4R_LAUNCH(false, false)
        }
#undef SMG_Q4R_LAUNCH
        return hipGetLastError();
    }
    g.part = part;
    g.nsplit = ns;
    g.part_ld = (uint32_t)((w.n + 7) / 8 * 8);
    if (w.mins && bf16)
        hipLaunchKernelGGL((gemm_q4r<true, true, 0, true>), dim3(tiles * ns), dim3(RNT), 0, s, g, ep);
    else if (w.mins)
        hipLaunchKernelGGL((gemm_q4r<true, true>), dim3(tiles * ns), dim3(RNT), 0, s, g, ep);
    else if (bf16)
        hipLaunchKernelGGL((gemm_q4r<false, true, 0, true>), dim3(tiles * ns), dim3(RNT), 0, s, g, ep);
    else
        hipLaunchKernelGGL((gemm_q4r<false, true>), dim3(tiles * ns), dim3(RNT), 0, s, g, ep);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t rtiles = (uint32_t)(((m + QR_BM - 1) / QR_BM) * ((w.n + QR_BN - 1) / QR_BN));
    if (bf16)
        hipLaunchKernelGGL(q4r_reduce<true>, dim3(rtiles), dim3(QR_NT), 0, s, g, ep);
    else
        hipLaunchKernelGGL(q4r_reduce<false>, dim3(rtiles), dim3(QR_NT), 0, s, g, ep);
    return hipGetLastError();
}

// The gate/up GEMM of a GatedLinear with glu at the store: w holds 8 gate then
// 8 up columns a group (n = 16 * ceil(nh / 8)); dst [m][nh] f16 gets
// glu(gate) * up, the values glu_rows (tile8) computes from the f16 GEMM
// output. One pass, no split: the caller takes it when q4r_nsplit is 1.
hipError_t launch_q4r_glu(const WDev &w, size_t m, uint16_t *dst, size_t nh, const uint16_t *lhs, uint32_t act,
                          hipStream_t s) {
    if (w.n != 16 * ((nh + 7) / 8) || w.mins) return hipErrorInvalidValue;  // a gated MLP's weights are Q4_0
    RArgs g = q4r_args(w, m, dst, 1, (long)nh, lhs, (long)w.k, 1.0f);
    g.act = act;
    g.nh = (uint32_t)nh;
    const uint32_t tiles = (uint32_t)(((m + RBM - 1) / RBM) * ((w.n + RBN - 1) / RBN));
    hipLaunchKernelGGL((gemm_q4r<false, false, 4, false>), dim3(tiles), dim3(RNT), 0, s, g, EpArgs{});
    return hipGetLastError();
}

// y [m][n] f32 += the f16 product of lhs [m][k] f16 and w, rounded as
// launch_q4r stores it: the split-K GEMM, with the residual add in its reduce.
// part: q4r_split_bytes(w, m) bytes, which must be nonzero (a split call).
hipError_t launch_q4r_resid(const WDev &w, size_t m, const uint16_t *lhs, float *y, float *part, size_t part_bytes,
                            hipStream_t s) {
    const size_t slice_bytes = m * ((w.n + 7) / 8 * 8) * sizeof(float);
    const uint32_t ns = part ? (uint32_t)std::min<size_t>(q4r_nsplit(w, m), part_bytes / slice_bytes) : 1;
    if (ns <= 1) return hipErrorInvalidValue;
    RArgs g = q4r_args(w, m, nullptr, 1, (long)w.n, lhs, (long)w.k, 1.0f);
    g.part = part;
    g.nsplit = ns;
    g.part_ld = (uint32_t)((w.n + 7) / 8 * 8);
    g.resid = y;
    const uint32_t tiles = (uint32_t)(((m + RBM - 1) / RBM) * ((w.n + RBN - 1) / RBN));
    const EpArgs ep = {};
    if (w.mins)
        hipLaunchKernelGGL((gemm_q4r<true, true>), dim3(tiles * ns), dim3(RNT), 0, s, g, ep);
    else
        hipLaunchKernelGGL((gemm_q4r<false, true>), dim3(tiles * ns), dim3(RNT), 0, s, g, ep);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t rtiles = (uint32_t)(((m + QR_BM - 1) / QR_BM) * ((w.n + QR_BN - 1) / QR_BN));
    hipLaunchKernelGGL(q4r_reduce<false>, dim3(rtiles), dim3(QR_NT), 0, s, g, ep);
    return hipGetLastError();
}

}  // namespace smg
