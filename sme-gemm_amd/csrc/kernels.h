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

// Rows at or below which the Q4 path runs the GEMV kernel.
constexpr size_t Q4_GEMV_MAX_ROWS = 8;

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
// (only used when the block is too large to quantize in-kernel).
size_t lowbit_scratch_bytes(const WDev &w, size_t m);
hipError_t launch_lowbit_gemv(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                              const EpArgs &ep, void *scratch, hipStream_t s);

// MFMA GEMM over any weight kind (Q4 / Q2 / Q1 dequantized to f16/bf16 in LDS,
// or dense), C[i,j] at dst[i*rs + j*cs] = ep(to16(beta * acc)).
hipError_t launch_gemm(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                       const uint16_t *lhs, long lhs_cs, long lhs_rs, float beta,
                       const EpArgs &ep, bool bf16, hipStream_t s);

// Q4 x f16 GEMM with register-resident weights (gemm_q4r.hip): f16, block >=
// 32, K a multiple of 64, row-major 16-byte-aligned A. launch_gemm uses it
// whenever q4r_supported holds.
bool q4r_supported(const WDev &w, size_t m, long lhs_cs, long lhs_rs, const uint16_t *lhs, bool bf16);
hipError_t launch_q4r(const WDev &w, size_t m, uint16_t *dst, long dst_cs, long dst_rs,
                      const uint16_t *lhs, long lhs_rs, float beta, const EpArgs &ep, hipStream_t s);

// Device-side repacks / dequant.
hipError_t launch_q4_dequant_dense(const WDev &q4, uint16_t *dense, bool to_bf16,
                                   hipStream_t s);

// dst[r][j] = (map[j] bit 30 ? src1 : src0)[r][map[j] & 0x3FFFFFFF], cells of
// cell_bytes (2, 16 or 64) in [rows][pad] arrays; map[j] < 0 writes zeros.
hipError_t launch_gather_columns(void *dst, size_t dst_pad, const void *src0, const void *src1,
                                 size_t src_pad, const int32_t *map, size_t rows, size_t cell_bytes,
                                 hipStream_t s);

// Sets the calling thread's smg_last_error() text and returns code.
int report(int code, const char *what);

}  // namespace smg
