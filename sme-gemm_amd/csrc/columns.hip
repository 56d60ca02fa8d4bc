// Column gathers over the device weight layouts (load-time repacks):
//   Q4Weights::permute_columns (src/kernels/q4/weights.rs:125-163)
//   Q1Weights::interleave      (src/kernels/lowbit/q1.rs:146-185)
//
// Every device array of a weight set is a [rows][n_pad] grid (common.cuh) of
// fixed-size cells (common.cuh): a Q4 chunk (16 B), a Q2/Q1 lane group of four
// 16-byte quarters (64 B), a scale or a min (2 B). Moving a column moves its
// cells unchanged, so the result is exact. Each thread copies one 16-byte unit
// (or one 2-byte scale); a wave covers consecutive columns of one row, read
// and written in runs wherever the map keeps consecutive columns together
// (the gate/up interleave keeps runs of 32).
#include "kernels.h"

namespace smg {

namespace {

// map[j] = source column of destination column j, bit 30 set when it comes
// from src1; -1 for the padding columns (written as zeros).
template <class T, int UNITS>
__global__ __launch_bounds__(256) void gather_cells(T *__restrict__ dst, size_t dst_pad,
                                                    const T *__restrict__ src0,
                                                    const T *__restrict__ src1, size_t src_pad,
                                                    const int32_t *__restrict__ map, size_t rows) {
    const size_t per_row = dst_pad * UNITS, total = rows * per_row;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (size_t)gridDim.x * blockDim.x) {
        const size_t r = t / per_row, x = t % per_row, j = x / UNITS, u = x % UNITS;
        const int32_t m = map[j];
        T v{};
        if (m >= 0) {
            const T *src = (m & (1 << 30)) ? src1 : src0;
            v = src[cell_index(r, (size_t)(m & ((1 << 30) - 1)), rows, src_pad) * UNITS + u];
        }
        dst[cell_index(r, j, rows, dst_pad) * UNITS + u] = v;
    }
}

template <class T, int UNITS>
hipError_t launch(void *dst, size_t dst_pad, const void *src0, const void *src1, size_t src_pad,
                  const int32_t *map, size_t rows, hipStream_t s) {
    const size_t total = rows * dst_pad * UNITS;
    if (!total) return hipSuccess;
    const size_t blocks = std::min<size_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL((gather_cells<T, UNITS>), dim3((unsigned)blocks), dim3(256), 0, s, (T *)dst,
                       dst_pad, (const T *)src0, (const T *)src1, src_pad, map, rows);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gather_columns(void *dst, size_t dst_pad, const void *src0, const void *src1,
                                 size_t src_pad, const int32_t *map, size_t rows, size_t cell_bytes,
                                 hipStream_t s) {
    switch (cell_bytes) {
        case 2: return launch<uint16_t, 1>(dst, dst_pad, src0, src1, src_pad, map, rows, s);
        case 16: return launch<uint4, 1>(dst, dst_pad, src0, src1, src_pad, map, rows, s);
        case 64: return launch<uint4, 4>(dst, dst_pad, src0, src1, src_pad, map, rows, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace smg
