// Measurement probes for the benchmark: a plain streaming read (the HBM time
// floor a single launch of a given size meets on this device) and the shader
// clock (the shader clock counter against the constant-rate wall clock).
// Neither is part of the matmul path.
#include "kernels.h"

namespace smg {

namespace {

// One pass over `bytes` (a multiple of 16) with 16-byte loads, grid-strided,
// every word folded into one value so no load is dead; the fold is stored only
// when it matches an impossible pattern, so the kernel writes nothing.
__global__ void __launch_bounds__(256) stream_read(const uint4 *p, size_t n16, unsigned *sink) {
    uint32_t acc = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u && sink) sink[0] = acc;
}

// stream_read, then threads 0 .. nout - 1 of the grid each store the low 16
// bits of their fold to out[thread]: a read of the same bytes that also
// writes a GEMV-sized output.
__global__ void __launch_bounds__(256) stream_read_store(const uint4 *p, size_t n16, uint16_t *out, size_t nout) {
    uint32_t acc = 0;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (size_t i = tid; i < n16; i += (size_t)gridDim.x * blockDim.x) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (tid < nout) out[tid] = (uint16_t)acc;
}

// Thread 0 of one workgroup spins `iters` times, reading the shader clock
// (clock64) and the 100 MHz wall clock before and after.
__global__ void clock_probe(unsigned long long *out, unsigned iters) {
    if (threadIdx.x != 0) return;
    const unsigned long long c0 = clock64(), w0 = wall_clock64();
    unsigned long long x = c0;
    for (unsigned i = 0; i < iters; i++) x = x * 6364136223846793005ull + 1442695040888963407ull;
    const unsigned long long c1 = clock64(), w1 = wall_clock64();
    out[0] = c1 - c0;
    out[1] = w1 - w0;
    out[2] = x;  // keeps the loop
}

}  // namespace

hipError_t launch_stream_read(const void *p, size_t bytes, unsigned *sink, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n16 + 255) / 256, 256 * 8);
    hipLaunchKernelGGL(stream_read, dim3((uint32_t)blocks), dim3(256), 0, s, (const uint4 *)p, n16, sink);
    return hipGetLastError();
}

hipError_t launch_stream_read_store(const void *p, size_t bytes, uint16_t *out, size_t nout, hipStream_t s) {
    const size_t n16 = bytes / 16;
    const size_t blocks = std::max<size_t>(std::min<size_t>((n16 + 255) / 256, 256 * 8), (nout + 255) / 256);
    hipLaunchKernelGGL(stream_read_store, dim3((uint32_t)blocks), dim3(256), 0, s, (const uint4 *)p, n16, out, nout);
    return hipGetLastError();
}

hipError_t launch_clock_probe(unsigned long long *out, unsigned iters, hipStream_t s) {
    hipLaunchKernelGGL(clock_probe, dim3(1), dim3(64), 0, s, out, iters);
    return hipGetLastError();
}

}  // namespace smg
