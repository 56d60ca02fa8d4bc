// The library's host code (csrc/api.hip's argument checks and descriptor
// parsing, csrc/quantize.hip's load-time quantizers) under AddressSanitizer
// and UndefinedBehaviorSanitizer, on the CPU: built with the sanitizers on the
// host side only (hipcc -Xarch_host), so the device code is the ordinary build
// and no call here reaches a GPU -- every call is a quantizer, a descriptor
// check, or an entry point refusing its arguments before it touches a device.
// Each buffer is allocated at exactly the size the header documents.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/smegemm_gpu.h"

static unsigned lcg = 7u;
static float frand() {
    lcg = lcg * 1664525u + 1013904223u;
    return ((float)(lcg >> 8) / (float)(1u << 24)) * 2.0f - 1.0f;
}

#define CHECK(cond)                                                          \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::fprintf(stderr, "failed: %s (line %d)\n", #cond, __LINE__); \
            return 1;                                                        \
        }                                                                    \
    } while (0)

int main() {
    const size_t shapes[][2] = {{1, 1}, {5, 7}, {37, 70}, {130, 33}, {64, 257}};
    const size_t blocks[] = {16, 32, 64, 128};
    for (auto &sh : shapes) {
        const size_t n = sh[0], k = sh[1];
        std::vector<float> w(n * k);
        for (auto &x : w) x = frand();
        w[0] = 0.0f;
        for (size_t block : blocks) {
            const size_t nbk = (k + block - 1) / block;
            for (int layout = 0; layout < 2; layout++) {
                for (int affine = 0; affine < 2; affine++) {
                    std::vector<uint8_t> quants((k * n + 1) / 2);
                    std::vector<uint16_t> scales(n * nbk), mins(n * nbk);
                    CHECK(smg_q4_quantize(w.data(), layout, n, k, block, affine, quants.data(), scales.data(),
                                          affine ? mins.data() : nullptr) == SMG_OK);
                }
                const int8_t cb[4] = {-1, 0, 1, 0}, zero[4] = {0, 0, 0, 0};
                std::vector<uint8_t> codes((k * n + 3) / 4), signs((k * n + 7) / 8);
                std::vector<uint16_t> s2(n * nbk), s1(n * nbk);
                CHECK(smg_q2_quantize(w.data(), layout, n, k, block, cb, codes.data(), s2.data()) == SMG_OK);
                CHECK(smg_q2_quantize(w.data(), layout, n, k, block, zero, codes.data(), s2.data()) == SMG_EINVAL);
                CHECK(smg_q1_quantize(w.data(), layout, n, k, block, signs.data(), s1.data()) == SMG_OK);
            }
        }
        CHECK(smg_q4_quantize(w.data(), 0, n, k, 48, 0, nullptr, nullptr, nullptr) == SMG_EINVAL);
    }

    // epilogue descriptors: valid, too long, an operand node without a pointer
    std::vector<uint16_t> col(300), ten(300 * 4);
    EpNode nodes[SMG_MAX_EP_NODES + 1];
    std::memset(nodes, 0, sizeof nodes);
    nodes[0].op = EP_OP_ADD_COL;
    nodes[0].ptr = col.data();
    nodes[1].op = EP_OP_ADD_TENSOR;
    nodes[1].ptr = ten.data();
    nodes[2].op = EP_OP_ACT;
    nodes[2].aux = EP_ACT_SILU;
    ep_desc16 d = {3, nodes};
    CHECK(smg_ep_check(&d, 300) == SMG_OK);
    CHECK(smg_ep_check(nullptr, 300) == SMG_OK);
    nodes[1].ptr = nullptr;
    CHECK(smg_ep_check(&d, 300) == SMG_EINVAL);
    CHECK(std::strlen(smg_last_error()) > 0);
    nodes[1].ptr = ten.data();
    nodes[1].ld = 5;  // a TENSOR row stride below n
    CHECK(smg_ep_check(&d, 300) == SMG_EINVAL);
    for (int i = 0; i <= SMG_MAX_EP_NODES; i++) nodes[i].op = EP_OP_ADD_SCALAR;
    d.n_nodes = SMG_MAX_EP_NODES + 1;
    CHECK(smg_ep_check(&d, 300) == SMG_EINVAL);
    d.nodes = nullptr;
    d.n_nodes = 2;
    CHECK(smg_ep_check(&d, 300) == SMG_EINVAL);

    // entry points refusing their arguments before any device work
    uint16_t buf[64] = {0};
    CHECK(gemm_gpu_f16f16_q4(1, nullptr, buf, buf, nullptr) == SMG_EINVAL);
    CHECK(gemm_gpu_f16_q2(1, nullptr, buf, buf, nullptr) == SMG_EINVAL);
    CHECK(gemm_gpu_f16f16_run(3, 4, 2, buf, 1, 2, 0, buf, 1, 2, buf, 1, 4, 0, 0x3C00) == SMG_EINVAL);
    CHECK(gemm_gpu_b16b16_run(3, 4, 2, buf, -1, 4, 0, buf, 1, 2, buf, 1, 4, 0, 0x3F80) == SMG_EINVAL);
    CHECK(gemm_gpu_f16f16_run(0, 4, 2, buf, 1, 4, 0, buf, 1, 2, buf, 1, 4, 0, 0x3C00) == SMG_OK);
    CHECK(smg_weights_info(nullptr, nullptr, nullptr, nullptr, nullptr) == SMG_EINVAL);
    smg_kv_cache *cache = nullptr;
    CHECK(smg_kv_cache_create(6, 4, 64, 8, &cache) == SMG_EINVAL);  // heads not a multiple of kv_heads
    CHECK(smg_kv_cache_create(4, 2, 12, 8, &cache) == SMG_EINVAL);  // head_dim not a multiple of 8
    CHECK(gemm_gpu_f16f16_q4_single(1, 4096, 4096) == 1);
    std::puts("host asan ok");
    return 0;
}
