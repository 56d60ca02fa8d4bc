// The C ABI (include/smegemm_gpu.h): weight handles, host-pointer drop-ins for
// the reference's gemm_sme_* entry points, and device-pointer entry points.
//
// Error contract (the reference's, src/kernels/q4/matmul.rs:85-90): a non-zero
// return leaves the caller's output untouched -- results are copied back to
// the host only after the kernels and the stream have completed successfully.
#include <pthread.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "kernels.h"
#include "scratch_pool.h"

using namespace smg;

struct smg_weights {
    WDev d;
    int device;
    size_t bytes;
    std::vector<void *> allocs;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char *what, hipError_t e = hipSuccess) {
    g_err = what;
    if (e != hipSuccess) {
        g_err += ": ";
        g_err += hipGetErrorString(e);
    }
    return code;
}

#define HIP_TRY(call, code)                                        \
    do {                                                           \
        hipError_t e_ = (call);                                    \
        if (e_ != hipSuccess) return fail((code), #call, e_);      \
    } while (0)

bool is_pow2(size_t x) { return x != 0 && (x & (x - 1)) == 0; }
size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---- device presence -------------------------------------------------------
int g_avail = -1;
pthread_once_t g_avail_once = PTHREAD_ONCE_INIT;
void probe_avail() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        g_avail = 0;
        return;
    }
    hipDeviceProp_t p;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
        g_avail = 0;
        return;
    }
    g_avail = std::strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

// ---- per-thread stream + staging (the reference's thread_local scratch) ----
struct Ctx {
    hipStream_t stream = nullptr;
    int device = -1;
    void *buf = nullptr;
    size_t cap = 0;
    ~Ctx() {
        if (buf) (void)hipFree(buf);
        if (stream) (void)hipStreamDestroy(stream);
    }
};
thread_local Ctx g_ctx;

// hipMalloc, or a forced failure while the environment has
// SMG_TEST_FAIL_ALLOC=1: a test hook for the reference's contract that a call
// whose allocation fails returns non-zero and leaves its output untouched, so
// the caller takes its portable path (src/kernels/q4/matmul.rs:85-89). The
// variable is read at every allocation.
hipError_t dev_malloc(void **p, size_t bytes) {
    const char *f = std::getenv("SMG_TEST_FAIL_ALLOC");
    if (f && f[0] == '1') {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}

int ctx_for(int device, size_t bytes, Ctx **out) {
    Ctx &c = g_ctx;
    HIP_TRY(hipSetDevice(device), SMG_EHIP);
    if (c.device != device) {
        if (c.buf) (void)hipFree(c.buf);
        if (c.stream) (void)hipStreamDestroy(c.stream);
        c.buf = nullptr;
        c.cap = 0;
        c.stream = nullptr;
        HIP_TRY(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking), SMG_EHIP);
        c.device = device;
    }
    if (bytes > c.cap) {
        if (c.buf) (void)hipFree(c.buf);
        c.buf = nullptr;
        c.cap = 0;
        size_t want = round_up(bytes, 1 << 20);
        if (dev_malloc(&c.buf, want) != hipSuccess) return fail(SMG_ENOMEM, "staging hipMalloc");
        c.cap = want;
    }
    *out = &c;
    return SMG_OK;
}

// ---- device-pointer scratch ---------------------------------------------------
// The *_dev entry points return before their kernels run, and a HIP graph may
// replay those kernels later still, so their scratch is never the thread's
// host-call staging buffer (freed when it grows): it comes from a grow-only
// pool keyed by (device, stream) whose outgrown buffers are retired, not freed.
struct HipDevAlloc {
    void *acquire(int device, size_t bytes) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return nullptr;
        if (cur != device && hipSetDevice(device) != hipSuccess) return nullptr;
        void *p = nullptr;
        const bool ok = dev_malloc(&p, bytes) == hipSuccess;
        if (cur != device) (void)hipSetDevice(cur);
        return ok ? p : nullptr;
    }
    void release(int, void *) {}  // the pool lives until the process ends
};
ScratchPool<HipDevAlloc> &dev_pool() {
    static ScratchPool<HipDevAlloc> *p = new ScratchPool<HipDevAlloc>();  // never destroyed
    return *p;
}

// ---- allocation-free scratch (smg_lowbit_matmul_dev_noalloc) --------------------
// One static array per device: the device keeps its copy until the process
// ends. In host code `scratch` is only a stand-in for the symbol, not a device
// address: kernels are given the address hipGetSymbolAddress returns for the
// current device, looked up once per device at that device's first call.
constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<void *> g_noalloc_ptr[NOALLOC_MAX_DEVICES];
std::mutex g_noalloc_mu;

}  // namespace

static __device__ __align__(256) uint8_t scratch[SMG_NOALLOC_SCRATCH_BYTES];

namespace {

// The device address of `device`'s copy of `scratch` into *out (looked up with
// that device current, the caller's device restored).
int noalloc_scratch(int device, void **out) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES)
        return fail(SMG_EINVAL, "smg_lowbit_matmul_dev_noalloc: device ordinal beyond the per-device table");
    void *p = g_noalloc_ptr[device].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_noalloc_mu);
        p = g_noalloc_ptr[device].load(std::memory_order_relaxed);
        if (!p) {
            int cur = -1;
            hipError_t e = hipGetDevice(&cur);
            if (e == hipSuccess && cur != device) e = hipSetDevice(device);
            if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (cur >= 0 && cur != device) (void)hipSetDevice(cur);
            if (e != hipSuccess || !p)
                return fail(SMG_EHIP, "smg_lowbit_matmul_dev_noalloc: hipGetSymbolAddress(scratch)", e);
            g_noalloc_ptr[device].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return SMG_OK;
}

bool trace_on() {
    static int on = -1;
    if (on < 0) {
        const char *e = std::getenv("SMEGEMM_TRACE");
        on = (e && *e && std::strcmp(e, "0") != 0) ? 1 : 0;
    }
    return on == 1;
}

// ---- epilogue marshalling --------------------------------------------------
bool op_is_row(uint32_t op) {
    return op == EP_OP_ADD_ROW || op == EP_OP_MUL_ROW || op == EP_OP_SUB_ROW ||
           op == EP_OP_DIV_ROW || op == EP_OP_MAX_ROW || op == EP_OP_MIN_ROW;
}
bool op_is_col(uint32_t op) {
    return op == EP_OP_ADD_COL || op == EP_OP_MUL_COL || op == EP_OP_SUB_COL ||
           op == EP_OP_DIV_COL || op == EP_OP_MAX_COL || op == EP_OP_MIN_COL;
}
bool op_is_tensor(uint32_t op) {
    return op == EP_OP_ADD_TENSOR || op == EP_OP_MUL_TENSOR || op == EP_OP_SUB_TENSOR ||
           op == EP_OP_DIV_TENSOR || op == EP_OP_MAX_TENSOR || op == EP_OP_MIN_TENSOR;
}
// Elements a node's operand spans (0 for scalar / act nodes).
size_t operand_elems(const EpNode &nd, size_t m, size_t n) {
    if (op_is_row(nd.op)) return m;
    if (op_is_col(nd.op)) return n;
    if (op_is_tensor(nd.op)) {
        size_t ld = nd.ld == 0 ? n : nd.ld;
        return m == 0 ? 0 : (m - 1) * ld + n;
    }
    return 0;
}

// The graph's nodes for the kernels: up to EP_FUSED in `fused`, which the
// product kernel's store applies, a longer graph in `tail`, which
// launch_ep_tail applies as a pass over C after a store with no graph. The
// Rust side validates operand lengths (validate_ep, src/exec/guard.rs:112-147);
// what this C boundary can check without lengths it checks here: known ops and
// activations, an operand pointer on every ROW / COL / TENSOR node (a kernel
// would read address 0 otherwise), and a TENSOR row stride of at least n.
struct EpPlan {
    EpArgs fused;
    EpLong tail;
    uint32_t count() const { return fused.n_nodes + tail.n_nodes; }
    const EpNode *nodes() const { return tail.n_nodes ? tail.nodes : fused.nodes; }
    EpNode *nodes() { return tail.n_nodes ? tail.nodes : fused.nodes; }
};

int ep_plan(const ep_desc16 *ep, EpPlan *p, size_t n, bool allow_tail = true) {
    std::memset(p, 0, sizeof(*p));
    if (!ep || ep->n_nodes == 0) return SMG_OK;
    if (ep->n_nodes > SMG_MAX_EP_NODES) return fail(SMG_EINVAL, "epilogue has too many nodes");
    if (ep->n_nodes > (uint32_t)EP_FUSED && !allow_tail)
        return fail(SMG_EINVAL, "this call applies at most SMG_FUSED_EP_NODES epilogue nodes");
    if (!ep->nodes) return fail(SMG_EINVAL, "epilogue has n_nodes > 0 and no node array");
    const bool tail = ep->n_nodes > (uint32_t)EP_FUSED;
    EpNode *nodes = tail ? p->tail.nodes : p->fused.nodes;
    uint32_t *fam = tail ? p->tail.fam : p->fused.fam, *cls = tail ? p->tail.cls : p->fused.cls;
    for (uint32_t i = 0; i < ep->n_nodes; i++) {
        const EpNode &nd = ep->nodes[i];
        if (ep_family(nd.op) == EPF_NONE) return fail(SMG_EINVAL, "epilogue node has an unknown op");
        if (nd.op == EP_OP_ACT && nd.aux > EP_ACT_GELU_EXACT)
            return fail(SMG_EINVAL, "epilogue node has an unknown activation");
        if ((op_is_row(nd.op) || op_is_col(nd.op) || op_is_tensor(nd.op)) && !nd.ptr)
            return fail(SMG_EINVAL, "epilogue row / col / tensor node has a null operand pointer");
        if (op_is_tensor(nd.op) && nd.ld != 0 && nd.ld < n)
            return fail(SMG_EINVAL, "epilogue tensor row stride is below n");
        nodes[i] = nd;
        fam[i] = ep_family(nd.op);
        cls[i] = ep_class(nd.op);
    }
    (tail ? p->tail.n_nodes : p->fused.n_nodes) = ep->n_nodes;
    return SMG_OK;
}

// After a product stored without a graph: the plan's tail, if it has one,
// over the m x n C at dst (row stride rs, column stride cs).
hipError_t plan_tail(const EpPlan &p, uint16_t *dst, long cs, long rs, size_t m, size_t n, bool bf16,
                     hipStream_t s) {
    return p.tail.n_nodes ? launch_ep_tail(dst, rs, cs, dst, rs, cs, m, n, 0.0f, false, p.tail, bf16, s)
                          : hipSuccess;
}

// ---- weight creation ---------------------------------------------------------
int alloc_dev(smg_weights *w, size_t bytes, void **p) {
    if (dev_malloc(p, bytes ? bytes : 16) != hipSuccess) return fail(SMG_ENOMEM, "weights hipMalloc");
    w->allocs.push_back(*p);
    w->bytes += bytes;
    return SMG_OK;
}

void destroy(smg_weights *w) {
    if (!w) return;
    if (w->device >= 0) (void)hipSetDevice(w->device);
    for (void *p : w->allocs) (void)hipFree(p);
    delete w;
}

int upload(smg_weights *w, const void *host, size_t bytes, void **dev) {
    int rc = alloc_dev(w, bytes, dev);
    if (rc) return rc;
    if (bytes) HIP_TRY(hipMemcpy(*dev, host, bytes, hipMemcpyHostToDevice), SMG_EHIP);
    return SMG_OK;
}

smg_weights *new_weights(int kind, size_t n, size_t k, size_t block) {
    smg_weights *w = new smg_weights();
    std::memset(&w->d, 0, sizeof(w->d));
    w->d.kind = kind;
    w->d.n = n;
    w->d.k = k;
    w->d.block = block;
    w->d.n_pad = round_up(n ? n : 1, 128);
    w->bytes = 0;
    (void)hipGetDevice(&w->device);
    return w;
}

// Nibble accessors for the two Q4 input formats.
struct Q4RowMajor {
    const uint8_t *q;
    size_t n;
    uint8_t operator()(size_t d, size_t j) const {
        size_t idx = d * n + j;
        return idx % 2 == 0 ? (q[idx / 2] & 0x0f) : (q[idx / 2] >> 4);
    }
};
struct Q4Band {  // q4/weights.rs:89-101 (128-column bands, 64 bytes a depth)
    const uint8_t *q;
    size_t k;
    uint8_t operator()(size_t d, size_t j) const {
        size_t b = j / 128, c = j % 128;
        uint8_t byte = q[b * k * 64 + d * 64 + c / 2];
        return (byte >> (4 * (c % 2))) & 0x0f;
    }
};

template <class Get>
int make_q4(Get get, const uint16_t *scales_rm, const uint16_t *mins_rm, const uint16_t *scales_band,
            const uint16_t *mins_band, size_t n, size_t k, size_t block, smg_weights **out) {
    if (!is_pow2(block)) return fail(SMG_EINVAL, "q4 block size must be a power of two");
    smg_weights *w = new_weights(W_Q4, n, k, block);
    WDev &d = w->d;
    d.nchunks = (k + Q4_CHUNK - 1) / Q4_CHUNK;
    const size_t nbk = (k + block - 1) / block;
    // rows for every depth the kernels may touch: the GEMM steps K in 64s
    d.sc_rows = std::max(nbk, (round_up(d.nchunks * Q4_CHUNK, 64) + block - 1) / block);
    d.k_pad = round_up(k ? k : 1, 64);
    std::vector<uint8_t> nib(cell_grid_rows(d.nchunks) * d.n_pad * 16, 0);
    for (size_t dd = 0; dd < k; dd++) {
        const size_t kc = dd / 32, x = dd % 32, wd = x / 8, e = (x % 8) / 2, h = x % 2;
        const size_t bitpos = 16 * h + 4 * e;
        const size_t byteoff = wd * 4 + bitpos / 8;
        const int shift = bitpos % 8;
        for (size_t j = 0; j < n; j++)
            nib[cell_index(kc, j, d.nchunks, d.n_pad) * 16 + byteoff] |= (uint8_t)((get(dd, j) ^ 8) << shift);
    }
    std::vector<uint16_t> sc(cell_grid_rows(d.sc_rows) * d.n_pad, 0), mn;
    const bool affine = mins_rm || mins_band;
    if (affine) mn.assign(cell_grid_rows(d.sc_rows) * d.n_pad, 0);
    for (size_t j = 0; j < n; j++)
        for (size_t b = 0; b < nbk; b++) {
            size_t src;
            if (scales_rm) {
                src = j * nbk + b;
                sc[cell_index(b, j, d.sc_rows, d.n_pad)] = scales_rm[src];
                if (affine) mn[cell_index(b, j, d.sc_rows, d.n_pad)] = mins_rm[src];
            } else {
                src = (j / 128) * (nbk * 128) + b * 128 + j % 128;
                sc[cell_index(b, j, d.sc_rows, d.n_pad)] = scales_band[src];
                if (affine) mn[cell_index(b, j, d.sc_rows, d.n_pad)] = mins_band[src];
            }
        }
    void *p;
    int rc;
    if ((rc = upload(w, nib.data(), nib.size(), &p))) { destroy(w); return rc; }
    d.codes = (const uint8_t *)p;
    if ((rc = upload(w, sc.data(), sc.size() * 2, &p))) { destroy(w); return rc; }
    d.scales = (const uint16_t *)p;
    if (affine) {
        if ((rc = upload(w, mn.data(), mn.size() * 2, &p))) { destroy(w); return rc; }
        d.mins = (const uint16_t *)p;
    }
    *out = w;
    return SMG_OK;
}

// Low-bit value accessors (2-bit code or 1-bit sign at depth d, column j).
struct Q2RowMajor {  // q2.rs:43-47
    const uint8_t *q;
    size_t n;
    uint8_t operator()(size_t d, size_t j) const {
        size_t idx = d * n + j;
        return (q[idx / 4] >> (2 * (idx % 4))) & 3;
    }
};
struct Q2Band {  // q2.rs:148-161
    const uint8_t *q;
    size_t band_bytes;
    uint8_t operator()(size_t d, size_t j) const {
        return (q[(j / 64) * band_bytes + (d / 4) * 64 + j % 64] >> (2 * (d % 4))) & 3;
    }
};
struct Q1RowMajor {  // q1.rs:35-41
    const uint8_t *q;
    size_t n, k;
    int inout;
    uint8_t operator()(size_t d, size_t j) const {
        size_t idx = inout ? d * n + j : j * k + d;
        return (q[idx / 8] >> (idx % 8)) & 1;
    }
};
struct Q1Band {  // q1.rs:186-201
    const uint8_t *q;
    size_t band_bytes;
    uint8_t operator()(size_t d, size_t j) const {
        size_t c = j % 64;
        size_t byte = (j / 64) * band_bytes + (d / 4) * 32 + c / 2;
        return (q[byte] >> (4 * (c % 2) + d % 4)) & 1;
    }
};

size_t lb_scale_index(size_t sc_per_band, size_t blk, size_t j) {  // q2.rs:17-20
    size_t c = j % 64;
    return (j / 64) * sc_per_band + blk * 64 + (c / 32) * 32 + 2 * (c % 16) + (c % 32) / 16;
}

template <class Get>
int make_lowbit(int kind, Get get, const uint16_t *scales, bool band_scales,
                const int8_t *codebook, size_t n, size_t k, size_t block, smg_weights **out) {
    if (!is_pow2(block) || block < 16 || block > 65536)
        return fail(SMG_EINVAL, "low-bit block size must be a power of two from 16 to 65536");
    smg_weights *w = new_weights(kind, n, k, block);
    WDev &d = w->d;
    const size_t grp = kind == W_Q2 ? Q2_GROUP : Q1_GROUP;
    d.nchunks = (k + grp - 1) / grp;  // lane groups along K
    const size_t nbk = (k + block - 1) / block;
    d.sc_rows = std::max(nbk, (d.nchunks * grp + block - 1) / block);
    d.k_pad = round_up(k ? k : 1, 64);
    if (kind == W_Q2)
        d.codebook = (uint32_t)(uint8_t)codebook[0] | ((uint32_t)(uint8_t)codebook[1] << 8) |
                     ((uint32_t)(uint8_t)codebook[2] << 16) | ((uint32_t)(uint8_t)codebook[3] << 24);
    std::vector<uint8_t> codes(cell_grid_rows(d.nchunks) * d.n_pad * 64, 0);
    for (size_t dd = 0; dd < k; dd++) {
        const uint32_t bit = kind == W_Q2 ? lb_bit<2>(dd) : lb_bit<1>(dd);
        for (size_t j = 0; j < n; j++) {
            const size_t off = kind == W_Q2 ? lb_dword_offset<2>(dd, j, d.nchunks, d.n_pad)
                                            : lb_dword_offset<1>(dd, j, d.nchunks, d.n_pad);
            codes[off + bit / 8] |= (uint8_t)(get(dd, j) << (bit % 8));
        }
    }
    std::vector<uint16_t> sc(cell_grid_rows(d.sc_rows) * d.n_pad, 0);
    for (size_t j = 0; j < n; j++)
        for (size_t b = 0; b < nbk; b++)
            sc[cell_index(b, j, d.sc_rows, d.n_pad)] =
                band_scales ? scales[lb_scale_index(nbk * 64, b, j)] : scales[j * nbk + b];
    void *p;
    int rc;
    if ((rc = upload(w, codes.data(), codes.size(), &p))) { destroy(w); return rc; }
    d.codes = (const uint8_t *)p;
    if ((rc = upload(w, sc.data(), sc.size() * 2, &p))) { destroy(w); return rc; }
    d.scales = (const uint16_t *)p;
    *out = w;
    return SMG_OK;
}

int make_dense(int kind, const uint16_t *rhs, size_t n, size_t k, long rs, long cs,
               smg_weights **out) {
    smg_weights *w = new_weights(kind, n, k, 0);
    WDev &d = w->d;
    d.k_pad = round_up(k ? k : 1, 64);
    std::vector<uint16_t> buf(d.n_pad * d.k_pad, 0);
    for (size_t j = 0; j < n; j++)
        for (size_t l = 0; l < k; l++) buf[j * d.k_pad + l] = rhs[(long)l * rs + (long)j * cs];
    void *p;
    int rc = upload(w, buf.data(), buf.size() * 2, &p);
    if (rc) { destroy(w); return rc; }
    d.dense = (const uint16_t *)p;
    *out = w;
    return SMG_OK;
}

// ---- one host-pointer call ---------------------------------------------------
// Stages lhs and epilogue operands, runs `launch` on the thread's stream, and
// copies dst back only after everything succeeded.
template <class Launch>
int host_call(const char *name, int device, size_t m, size_t n, size_t k, uint16_t *dst,
              size_t dst_elems, bool preload_dst, const uint16_t *lhs, size_t lhs_elems,
              const ep_desc16 *ep, size_t extra_scratch, Launch launch) {
    EpPlan plan;
    int rc = ep_plan(ep, &plan, n);
    if (rc) return rc;
    EpNode *nodes = plan.nodes();
    const uint32_t nn = plan.count();
    size_t op_elems[SMG_MAX_EP_NODES] = {0};
    size_t total = round_up(lhs_elems * 2, 256) + round_up(dst_elems * 2, 256) +
                   round_up(extra_scratch, 256);
    for (uint32_t i = 0; i < nn; i++) {
        op_elems[i] = nodes[i].ptr ? operand_elems(nodes[i], m, n) : 0;
        total += round_up(op_elems[i] * 2, 256);
    }
    Ctx *c;
    if ((rc = ctx_for(device, total, &c))) return rc;
    uint8_t *p = (uint8_t *)c->buf;
    uint16_t *d_lhs = (uint16_t *)p;
    p += round_up(lhs_elems * 2, 256);
    uint16_t *d_dst = (uint16_t *)p;
    p += round_up(dst_elems * 2, 256);
    void *scratch = p;
    p += round_up(extra_scratch, 256);
    for (uint32_t i = 0; i < nn; i++) {
        if (!op_elems[i]) continue;
        HIP_TRY(hipMemcpyAsync(p, nodes[i].ptr, op_elems[i] * 2, hipMemcpyHostToDevice,
                               c->stream), SMG_EHIP);
        nodes[i].ptr = p;
        p += round_up(op_elems[i] * 2, 256);
    }
    if (lhs_elems)
        HIP_TRY(hipMemcpyAsync(d_lhs, lhs, lhs_elems * 2, hipMemcpyHostToDevice, c->stream),
                SMG_EHIP);
    if (preload_dst && dst_elems)
        HIP_TRY(hipMemcpyAsync(d_dst, dst, dst_elems * 2, hipMemcpyHostToDevice, c->stream),
                SMG_EHIP);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    const bool tr = trace_on();
    if (tr) {
        (void)hipEventCreate(&e0);
        (void)hipEventCreate(&e1);
        (void)hipEventRecord(e0, c->stream);
    }
    hipError_t e = launch(d_dst, d_lhs, plan, scratch, c->stream);
    if (e != hipSuccess) return fail(SMG_EHIP, name, e);
    if (tr) (void)hipEventRecord(e1, c->stream);
    HIP_TRY(hipStreamSynchronize(c->stream), SMG_EHIP);
    if (tr) {
        float ms = 0;
        (void)hipEventElapsedTime(&ms, e0, e1);
        std::fprintf(stderr, "[smegemm] %s %zux%zux%zu %.1f us\n", name, m, n, k, ms * 1e3);
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
    }
    if (dst_elems)
        HIP_TRY(hipMemcpy(dst, d_dst, dst_elems * 2, hipMemcpyDeviceToHost), SMG_EHIP);
    return SMG_OK;
}

// ---- one host-slice call of a model part -----------------------------------------
// A host array of a model part's call: `in` is copied to the device before
// the part runs, `out` back after it finished without error.
struct Slice {
    void *host;
    size_t bytes;
    bool in, out;
};

// n * elems * width bytes, or false when the product overflows.
bool slice_bytes(size_t n, size_t elems, size_t width, size_t *out) {
    size_t t;
    return !__builtin_mul_overflow(n, elems, &t) && !__builtin_mul_overflow(t, width, out);
}

// Stages the slices in the thread's staging buffer, runs `run(dev, stream)`
// (the part's device form over the staged pointers, null where the host one
// is null) on the thread's stream, waits, and copies the written slices back
// only when it succeeded: on an error they are untouched.
template <size_t N, class Run>
int slice_call(int device, Slice (&s)[N], Run run) {
    size_t total = 256;
    for (const Slice &x : s) total += round_up(x.bytes, 256);
    Ctx *c;
    int rc = ctx_for(device, total, &c);
    if (rc) return rc;
    void *d[N];
    uint8_t *p = (uint8_t *)c->buf;
    for (size_t i = 0; i < N; i++) {
        d[i] = s[i].host ? p : nullptr;
        if (s[i].host && s[i].in && s[i].bytes)
            HIP_TRY(hipMemcpyAsync(p, s[i].host, s[i].bytes, hipMemcpyHostToDevice, c->stream), SMG_EHIP);
        p += round_up(s[i].bytes, 256);
    }
    rc = run(d, (void *)c->stream);
    const hipError_t e = hipStreamSynchronize(c->stream);
    if (rc) return rc;
    if (e != hipSuccess) return fail(SMG_EHIP, "hipStreamSynchronize", e);
    for (size_t i = 0; i < N; i++)
        if (s[i].host && s[i].out && s[i].bytes)
            HIP_TRY(hipMemcpyAsync(s[i].host, d[i], s[i].bytes, hipMemcpyDeviceToHost, c->stream), SMG_EHIP);
    HIP_TRY(hipStreamSynchronize(c->stream), SMG_EHIP);
    return SMG_OK;
}

int check_kind(const smg_weights *w, int kind) {
    if (!w) return fail(SMG_EINVAL, "null weights");
    if (w->d.kind != kind) return fail(SMG_EKIND, "weight handle of another kind");
    return SMG_OK;
}

// A handle of n_out columns whose column j is column cols[j] of a, or of b when
// bit 30 of cols[j] is set. Every device array of a weight set is a
// [rows][n_pad] grid of cells (common.cuh), so whole cells move unchanged.
int gather_columns(const smg_weights *a, const smg_weights *b, const std::vector<int32_t> &cols,
                   smg_weights **out) {
    HIP_TRY(hipSetDevice(a->device), SMG_EHIP);
    const WDev &s = a->d;
    smg_weights *w = new_weights(s.kind, cols.size(), s.k, s.block);
    WDev &d = w->d;
    d.nchunks = s.nchunks;
    d.sc_rows = s.sc_rows;
    d.k_pad = s.k_pad;
    d.codebook = s.codebook;
    std::vector<int32_t> map(d.n_pad, -1);
    std::copy(cols.begin(), cols.end(), map.begin());
    int32_t *dmap = nullptr;
    hipError_t e = dev_malloc((void **)&dmap, map.size() * sizeof(int32_t));
    if (e != hipSuccess) { destroy(w); return fail(SMG_ENOMEM, "column map hipMalloc", e); }
    e = hipMemcpy(dmap, map.data(), map.size() * sizeof(int32_t), hipMemcpyHostToDevice);
    struct Field {
        const void *s0, *s1;
        const void **dst;
        size_t rows, cell;
    };
    const Field f[3] = {
        {s.codes, b ? b->d.codes : nullptr, (const void **)&d.codes, s.nchunks, s.kind == W_Q4 ? 16u : 64u},
        {s.scales, b ? b->d.scales : nullptr, (const void **)&d.scales, s.sc_rows, 2},
        {s.mins, b ? b->d.mins : nullptr, (const void **)&d.mins, s.sc_rows, 2}};
    int rc = SMG_OK;
    for (int i = 0; i < 3 && e == hipSuccess && rc == SMG_OK; i++) {
        if (!f[i].s0) continue;
        void *p;
        if ((rc = alloc_dev(w, cell_grid_rows(f[i].rows) * d.n_pad * f[i].cell, &p))) break;
        *f[i].dst = p;
        e = launch_gather_columns(p, d.n_pad, f[i].s0, f[i].s1, s.n_pad, dmap, f[i].rows, f[i].cell, nullptr);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    (void)hipFree(dmap);
    if (rc) { destroy(w); return rc; }
    if (e != hipSuccess) { destroy(w); return fail(SMG_EHIP, "column gather", e); }
    *out = w;
    return SMG_OK;
}

// The op-graph of rows r0.. of a call, for a launch whose row 0 is row r0:
// ROW operands advance by r0 values, TENSOR operands by r0 rows.
EpArgs ep_from_row(const EpArgs &ea, size_t r0, size_t n) {
    EpArgs out = ea;
    for (uint32_t i = 0; i < ea.n_nodes; i++) {
        EpNode &nd = out.nodes[i];
        if (op_is_row(nd.op)) nd.ptr = (const uint16_t *)nd.ptr + r0;
        if (op_is_tensor(nd.op)) nd.ptr = (const uint16_t *)nd.ptr + r0 * (nd.ld ? nd.ld : n);
    }
    return out;
}

// Q4 dispatch: the GEMV where q4_gemv_serves() (up to 8 rows, or 16 with a
// scale per chunk); up to Q4_GEMV_CHUNK_ROWS rows with a scale per chunk, the
// 16-row GEMV once per 16 rows (measured at K = 4096: 24 rows take 14 us
// there against 51 us in the unsplit GEMM, whose 128 x 256 tiles leave most
// compute units idle at N = 4096 to 14336); the MFMA GEMM above, K split over
// the compute units when its tiles are few and `split` (q4_split_bytes) is
// given.
// Without gemm_q4r (an A it cannot read: not 16-byte aligned) the calls above
// Q4_GEMV_CHUNK_ROWS go to gemm_kernel, whose 128 x 128 tiles are as few: at
// K = 4096 it took 115 us for any of 33-128 rows at N = 4096 or 14336, where
// 16-row GEMV launches take about 7.7 us (N = 4096) or 17.6 us (N = 14336)
// each. So those calls stay on the GEMV up to Q4_GEMV_CHUNK_MAX rows while
// (launches x N) stays within Q4_GEMV_CHUNK_COLS (N = 14336: up to 96 rows).
constexpr size_t Q4_GEMV_CHUNK_ROWS = 32, Q4_GEMV_CHUNK_MAX = 128, Q4_GEMV_CHUNK_COLS = 6 * 14336;
bool q4_gemv_rows(const WDev &w, size_t m, bool gemm_q4r) {
    if (q4_gemv_serves(w, m)) return true;
    if (!q4_gemv_serves(w, Q4_GEMV_WIDE_ROWS)) return false;
    if (m <= Q4_GEMV_CHUNK_ROWS) return true;
    return !gemm_q4r && m <= Q4_GEMV_CHUNK_MAX &&
           (m + Q4_GEMV_WIDE_ROWS - 1) / Q4_GEMV_WIDE_ROWS * w.n <= Q4_GEMV_CHUNK_COLS;
}
// Bytes of split-K partials a run_q4 call with this A will use: only calls that
// gemm_q4r serves (it reads A itself, so an A it cannot read goes elsewhere and
// needs none). lhs == nullptr stands for the host entry points' staging copy of
// A, which is 256-byte aligned.
size_t q4_split_bytes(const WDev &w, size_t m, const uint16_t *lhs, bool bf16) {
    if (!q4r_supported(w, m, 1, (long)w.k, lhs, bf16) || q4_gemv_rows(w, m, true)) return 0;
    return q4r_split_bytes(w, m);
}
hipError_t run_q4(const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs, const EpArgs &ea,
                  bool bf16, hipStream_t s, void *split, size_t split_bytes) {
    if (q4_gemv_serves(w, m)) return launch_q4_gemv(w, m, dst, lhs, ea, bf16, s);
    const bool q4r = q4r_supported(w, m, 1, (long)w.k, lhs, bf16);
    if (q4_gemv_rows(w, m, q4r)) {
        for (size_t r0 = 0; r0 < m; r0 += Q4_GEMV_WIDE_ROWS) {
            const size_t rows = std::min(Q4_GEMV_WIDE_ROWS, m - r0);
            const hipError_t e = launch_q4_gemv(w, rows, dst + r0 * w.n, lhs + r0 * w.k, ep_from_row(ea, r0, w.n),
                                                bf16, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (q4r) return launch_q4r(w, m, dst, 1, (long)w.n, lhs, (long)w.k, 1.0f, ea, (float *)split, split_bytes, bf16, s);
    return launch_gemm(w, m, dst, 1, (long)w.n, lhs, 1, (long)w.k, 1.0f, ea, bf16, s);
}

// Split-K partial sums for the device-pointer callers of run_q4: a pool of
// its own, so a buffer never aliases the dev_pool() scratch that the caller
// (the MLP, the decode entry points) may hold on the same stream.
ScratchPool<HipDevAlloc> &split_pool() {
    static ScratchPool<HipDevAlloc> *p = new ScratchPool<HipDevAlloc>();  // never destroyed
    return *p;
}
// SMG_ENOMEM for a failed allocation (the split-K partials), else SMG_EHIP.
int q4_fail(const char *what, hipError_t e) {
    if (e == hipErrorOutOfMemory) return fail(SMG_ENOMEM, (std::string(what) + ": split-K partials hipMalloc").c_str());
    return fail(SMG_EHIP, what, e);
}
hipError_t run_q4_dev(int device, const WDev &w, size_t m, uint16_t *dst, const uint16_t *lhs,
                      const EpArgs &ea, bool bf16, hipStream_t s) {
    const size_t sb = q4_split_bytes(w, m, lhs, bf16);
    void *part = nullptr;
    if (sb && !(part = split_pool().get(device, s, sb))) return hipErrorOutOfMemory;
    return run_q4(w, m, dst, lhs, ea, bf16, s, part, sb);
}

// y [m][w.n] f32 += the f16 projection of lhs (the residual add after an out
// or down projection): in the split-K reduce where run_q4 would split, else
// the f16 result into tmp16, then add_f16_values.
hipError_t q4_add_dev(int device, const WDev &w, size_t m, const uint16_t *lhs, uint16_t *tmp16, float *y,
                      hipStream_t s) {
    const size_t sb = q4_split_bytes(w, m, lhs, false);
    if (sb) {
        void *part = split_pool().get(device, s, sb);
        if (!part) return hipErrorOutOfMemory;
        return launch_q4r_resid(w, m, lhs, y, (float *)part, sb, s);
    }
    const hipError_t e = run_q4_dev(device, w, m, tmp16, lhs, EpArgs{}, false, s);
    return e != hipSuccess ? e : launch_add_f16(tmp16, m * w.n, y, s);
}

// k == 0: every output is the epilogue applied to +0 (reference GEMM of an
// empty sum); the GEMV and GEMM kernels handle it (zero chunks, zero steps).

float half_bits_to_float(uint16_t h, bool bf16) {
    if (bf16) {
        uint32_t u = (uint32_t)h << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
    // f16 -> f32 (exact)
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ffu, u;
    if (exp == 0x1f) u = sign | 0x7f800000u | (man << 13);
    else if (exp == 0) {
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    } else u = sign | ((exp + 112u) << 23) | (man << 13);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

// ---- decode block handles ------------------------------------------------------
struct smg_kv_cache {
    int device;
    size_t heads, kv_heads, hd, cap, len;
    float scale;
    uint16_t *k, *v;  // [cap][kv_heads * hd]
};

struct smg_attn {
    int device;
    smg_weights *qkv;  // columns in the fused store's order: tiles of RoPE pairs
    smg_weights *out;
    size_t heads, kv_heads, hd;
    double theta;      // 0: no RoPE
    std::vector<float> inv_freq;
    float *rope = nullptr;  // device: cos [rope_cap][hd/2], then sin [rope_cap][hd/2]
    size_t rope_cap = 0;
    std::vector<float *> retired;  // outgrown tables, kept: queued work may read them
    std::mutex mu;
};

struct smg_mlp {
    int device;
    smg_weights *up;  // gated: tiles of 8 gate + the same 8 up columns (zero-padded)
    smg_weights *down;
    uint32_t act;
    bool gated;
    size_t hidden;
};

struct smg_block {
    int device;
    float *norm1, *norm2;  // device f32 [d]
    float *bias1, *bias2;  // device f32 [d] or null (Norm::layer's bias)
    bool layer1, layer2;   // Norm::layer (else Norm::rms)
    size_t d;
    float eps1, eps2;
    smg_attn *attn;
    smg_mlp *mlp;
};

namespace {

// Device column p of an attention's qkv: tile p/16 of head p/hd holds columns
// 8q..8q+7 and hd/2+8q..hd/2+8q+7 (q = tile within the head), so each RoPE
// pair (i, i + hd/2) sits in one workgroup's tile (lanes c and c ^ 8).
std::vector<int32_t> qkv_store_order(size_t nq, size_t hd) {
    std::vector<int32_t> cols(nq);
    const size_t half = hd / 2;
    for (size_t p = 0; p < nq; p++) {
        const size_t head = p / hd, qt = (p % hd) / 16, cc = p % 16;
        cols[p] = (int32_t)(head * hd + (cc < 8 ? 8 * qt + cc : half + 8 * qt + cc - 8));
    }
    return cols;
}

// Device column order of a gated MLP's up: tiles of 8 gate columns then the
// same 8 up columns, from GatedLinear's interleave (32 gate, 32 up, ...; the
// last chunk w < 32 wide; src/linear.rs:601-619); past `hidden`, zero columns.
std::vector<int32_t> glu_store_order(size_t hidden) {
    const size_t tiles = (hidden + 7) / 8;
    std::vector<int32_t> cols(16 * tiles, -1);
    for (size_t j = 0; j < hidden; j++) {
        const size_t c0 = j / 32 * 32, w = std::min<size_t>(32, hidden - c0);
        cols[16 * (j / 8) + j % 8] = (int32_t)(2 * c0 + (j - c0));          // gate j
        cols[16 * (j / 8) + 8 + j % 8] = (int32_t)(2 * c0 + w + (j - c0));  // up j
    }
    return cols;
}

// The attention's RoPE table covering positions [0, cap): cos and sin of
// (pos as f32 * inv_freq[i]) in f32 (examples/bonsai/model.rs:77-85), computed
// here on the host as the reference computes its angles. A table that is
// outgrown is retired, not freed. *tab and *tab_cap receive the table and its
// capacity as read under the lock (another thread may grow the table after the
// lock is released, so a caller uses this snapshot, never a->rope / a->rope_cap).
int ensure_rope(smg_attn *a, size_t cap, const float **tab_out, size_t *tab_cap) {
    *tab_out = nullptr;
    *tab_cap = 0;
    if (a->theta <= 0.0) return SMG_OK;
    std::lock_guard<std::mutex> lk(a->mu);
    if (a->rope_cap >= cap) {
        *tab_out = a->rope;
        *tab_cap = a->rope_cap;
        return SMG_OK;
    }
    const size_t half = a->hd / 2, ncap = std::max(cap, 2 * a->rope_cap);
    std::vector<float> tab(2 * ncap * half);
    for (size_t pos = 0; pos < ncap; pos++)
        for (size_t i = 0; i < half; i++) {
            const float ang = (float)pos * a->inv_freq[i];
            tab[pos * half + i] = std::cos(ang);
            tab[ncap * half + pos * half + i] = std::sin(ang);
        }
    float *d = nullptr;
    HIP_TRY(hipSetDevice(a->device), SMG_EHIP);
    if (dev_malloc((void **)&d, tab.size() * 4) != hipSuccess) return fail(SMG_ENOMEM, "rope table hipMalloc");
    hipError_t e = hipMemcpy(d, tab.data(), tab.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return fail(SMG_EHIP, "rope table upload", e);
    }
    if (a->rope) a->retired.push_back(a->rope);
    a->rope = d;
    a->rope_cap = ncap;
    *tab_out = d;
    *tab_cap = ncap;
    return SMG_OK;
}

// One call's device scratch, carved from the stream's pool buffer.
struct DecodeScratch {
    uint16_t *q16, *att16, *h16, *hid;
    float *po;
    float2 *pml;
};
int decode_scratch(int device, void *stream, size_t qlen, size_t nsplit, size_t heads, size_t h16_elems,
                   size_t hid_elems, DecodeScratch *sc, size_t base = 0) {
    const size_t a = 256;
    const size_t sizes[6] = {round_up(qlen * 2, a), round_up(qlen * 2, a), round_up(h16_elems * 2, a),
                             round_up(hid_elems * 2, a), round_up(nsplit * qlen * 4, a),
                             round_up(nsplit * heads * 8, a)};
    size_t total = 0;
    for (size_t z : sizes) total += z;
    uint8_t *p = (uint8_t *)dev_pool().get(device, stream, base + total);
    if (!p) return fail(SMG_ENOMEM, "decode scratch hipMalloc");
    p += base;  // what a caller keeps below `base` stays untouched
    sc->q16 = (uint16_t *)p;
    p += sizes[0];
    sc->att16 = (uint16_t *)p;
    p += sizes[1];
    sc->h16 = (uint16_t *)p;
    p += sizes[2];
    sc->hid = (uint16_t *)p;
    p += sizes[3];
    sc->po = (float *)p;
    p += sizes[4];
    sc->pml = (float2 *)p;
    return SMG_OK;
}

int check_cache(const smg_attn *a, const smg_kv_cache *c, size_t rows) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (c->heads != a->heads || c->kv_heads != a->kv_heads || c->hd != a->hd)
        return fail(SMG_EINVAL, "the cache's heads match the block's");
    if (c->device != a->device) return fail(SMG_EINVAL, "the cache is on another device");
    if (c->len + rows > c->cap) return fail(SMG_EINVAL, "KvCache full: the rows do not fit in the cache");
    return SMG_OK;
}

// The attention half at one row: qkv (from x16, or the RMS norm of the f32 row
// nx with weights nw), RoPE and the cache append at the store, attention, out
// projection added into y. Appends the cache row.
int attn_step(smg_attn *a, smg_kv_cache *c, const uint16_t *x16, const float *nx, const float *nw, float eps,
              float *y, void *stream, size_t base = 0) {
    int rc = check_cache(a, c, 1);
    if (rc) return rc;
    const float *rope = nullptr;
    size_t rope_cap = 0;
    if ((rc = ensure_rope(a, c->cap, &rope, &rope_cap))) return rc;
    const size_t pos = c->len, ld = a->kv_heads * a->hd, qlen = a->heads * a->hd, half = a->hd / 2;
    const size_t nsplit = attn_splits(pos + 1);
    DecodeScratch sc;
    if ((rc = decode_scratch(a->device, stream, qlen, nsplit, a->heads, 0, 0, &sc, base))) return rc;
    hipStream_t s = (hipStream_t)stream;
    BlkArgs b = {};
    b.nx = nx;
    b.nw = nw;
    b.eps = eps;
    b.q_out = sc.q16;
    b.k_row = c->k + pos * ld;
    b.v_row = c->v + pos * ld;
    if (a->theta > 0.0) {
        b.cs = rope + pos * half;
        b.sn = rope + rope_cap * half + pos * half;
    }
    b.scale = c->scale;
    b.heads = (uint32_t)a->heads;
    b.kv_heads = (uint32_t)a->kv_heads;
    b.hd = (uint32_t)a->hd;
    hipError_t e = launch_blk_gemv(a->qkv->d, 1, x16, b, BS_QKV, nx != nullptr, s);
    if (e != hipSuccess) return fail(SMG_EHIP, "qkv projection", e);
    AttnArgs at = {};
    at.q = sc.q16;
    at.k = c->k;
    at.v = c->v;
    at.po = sc.po;
    at.pml = sc.pml;
    at.len = (uint32_t)(pos + 1);
    at.ld = (uint32_t)ld;
    at.hd = (uint32_t)a->hd;
    at.heads = (uint32_t)a->heads;
    at.group = (uint32_t)(a->heads / a->kv_heads);
    if ((e = launch_attention(at, sc.att16, true, s)) != hipSuccess) return fail(SMG_EHIP, "attention", e);
    BlkArgs r = {};
    r.x = y;
    if ((e = launch_blk_gemv(a->out->d, 1, sc.att16, r, BS_RESID, false, s)) != hipSuccess)
        return fail(SMG_EHIP, "out projection", e);
    c->len = pos + 1;
    return SMG_OK;
}

// Device scratch carved from the stream's pool above `base`: each size is
// rounded up to 256 bytes; the pointers come back in order.
int carve_scratch(int device, void *stream, size_t base, std::initializer_list<size_t> sizes, uint8_t **out) {
    size_t total = 0;
    for (size_t z : sizes) total += round_up(z, 256);
    uint8_t *p = (uint8_t *)dev_pool().get(device, stream, base + total);
    if (!p) return fail(SMG_ENOMEM, "scratch hipMalloc");
    p += base;
    size_t i = 0;
    for (size_t z : sizes) {
        out[i++] = p;
        p += round_up(z, 256);
    }
    return SMG_OK;
}

// The attention partial sums one launch may hold: a causal block of rows is
// attended in chunks of rows whose partials fit (row r of a chunk needs
// attn_splits(its prefix) x heads x (hd + 2) floats).
// A block of rows that runs the matrix-core form is one launch with no
// partials.
constexpr size_t ATT_PART_BYTES = 64u << 20;
size_t causal_chunk_rows(size_t rows, size_t last_len, size_t heads, size_t hd) {
    if (attn_rows_blocked(rows)) return rows;
    const size_t per_row = attn_partial_floats(1, last_len, heads, hd) * 4;
    return std::max<size_t>(1, std::min(rows, ATT_PART_BYTES / per_row));
}
size_t causal_part_bytes(size_t rows, size_t last_len, size_t heads, size_t hd) {
    if (attn_rows_blocked(rows)) return 0;
    return attn_partial_floats(causal_chunk_rows(rows, last_len, heads, hd), last_len, heads, hd) * 4;
}

// Causal attention of `rows` f16 query rows (q16 [rows][heads hd], already
// f16(q * scale)) over k / v whose row r attends to keys 0 .. start + r: one
// launch_attention per chunk of rows, partials in `part`
// (causal_chunk_rows(...) rows' worth).
hipError_t causal_attention(const uint16_t *q16, const uint16_t *k, const uint16_t *v, size_t start, size_t rows,
                            size_t heads, size_t kv_heads, size_t hd, float *part, void *out, bool f16_out,
                            hipStream_t s) {
    const size_t qlen = heads * hd, last = start + rows;
    const size_t rc = causal_chunk_rows(rows, last, heads, hd);
    const size_t po_floats = attn_rows_blocked(rows) ? 0 : rc * attn_splits(last) * heads * hd;
    for (size_t r0 = 0; r0 < rows; r0 += rc) {
        AttnArgs at = {};
        at.q = q16 + r0 * qlen;
        at.k = k;
        at.v = v;
        at.po = part;
        at.pml = (float2 *)(part + po_floats);
        at.len = (uint32_t)(start + r0 + 1);
        at.rows = (uint32_t)std::min(rc, rows - r0);
        at.ld = (uint32_t)(kv_heads * hd);
        at.hd = (uint32_t)hd;
        at.heads = (uint32_t)heads;
        at.group = (uint32_t)(heads / kv_heads);
        void *o = f16_out ? (void *)((uint16_t *)out + r0 * qlen) : (void *)((float *)out + r0 * qlen);
        const hipError_t e = launch_attention(at, o, f16_out, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// The attention half for m > 1 rows of x16 (SelfAttention::accumulate,
// self_attention.rs:148-240: qkv over all rows, every row's key and value
// appended, then attend_causal, then out): the qkv projection as one Q4 call
// over the rows (the GEMM past the GEMV's rows), qkv_rows for RoPE, the cache
// append and q's rounding at positions pos .. pos + m - 1, causal attention
// (row r over positions 0 .. pos + r, kv_attention.rs:155-240), and the out
// projection added into y (8-row GEMV launches adding in their store, or a
// GEMM and an add). Appends m cache rows.
int attn_rows(smg_attn *a, smg_kv_cache *c, const uint16_t *x16, float *y, size_t m, void *stream,
              size_t base = 0) {
    int rc = check_cache(a, c, m);
    if (rc) return rc;
    const float *rope = nullptr;
    size_t rope_cap = 0;
    if ((rc = ensure_rope(a, c->cap, &rope, &rope_cap))) return rc;
    const size_t pos = c->len, ld = a->kv_heads * a->hd, qlen = a->heads * a->hd, half = a->hd / 2;
    const size_t nq = a->qkv->d.n, d_out = a->out->d.n;
    uint8_t *bufs[5];
    if ((rc = carve_scratch(a->device, stream, base,
                            {m * nq * 2, m * qlen * 2, m * qlen * 2, m > 8 ? m * d_out * 2 : 0,
                             causal_part_bytes(m, pos + m, a->heads, a->hd)},
                            bufs)))
        return rc;
    uint16_t *qkv16 = (uint16_t *)bufs[0], *q16 = (uint16_t *)bufs[1], *att16 = (uint16_t *)bufs[2];
    uint16_t *out16 = (uint16_t *)bufs[3];
    float *part = (float *)bufs[4];
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = run_q4_dev(a->qkv->device, a->qkv->d, m, qkv16, x16, EpArgs{}, false, s);
    if (e != hipSuccess) return q4_fail("qkv projection", e);
    QkvRowsArgs qa = {};
    qa.qkv = qkv16;
    qa.q_out = q16;
    qa.k_cache = c->k + pos * ld;
    qa.v_cache = c->v + pos * ld;
    if (a->theta > 0.0) {
        qa.cs = rope + pos * half;
        qa.sn = rope + rope_cap * half + pos * half;
    }
    qa.scale = c->scale;
    qa.m = (uint32_t)m;
    qa.heads = (uint32_t)a->heads;
    qa.kv_heads = (uint32_t)a->kv_heads;
    qa.hd = (uint32_t)a->hd;
    if ((e = launch_qkv_rows(qa, s)) != hipSuccess) return fail(SMG_EHIP, "qkv rows", e);
    if ((e = causal_attention(q16, c->k, c->v, pos, m, a->heads, a->kv_heads, a->hd, part, att16, true, s)) !=
        hipSuccess)
        return fail(SMG_EHIP, "causal attention", e);
    if (m <= 8) {
        BlkArgs r = {};
        r.x = y;
        if ((e = launch_blk_gemv(a->out->d, m, att16, r, BS_RESID, false, s)) != hipSuccess)
            return fail(SMG_EHIP, "out projection", e);
    } else {
        if ((e = q4_add_dev(a->out->device, a->out->d, m, att16, out16, y, s)) != hipSuccess)
            return q4_fail("out projection", e);
    }
    c->len = pos + m;
    return SMG_OK;
}

// The MLP half: y += down(act(up(x))) for `rows` rows of x16, or (nx) of the
// norm of the f32 rows nx with weights nw: RMS (fused into the gate/up GEMV for
// one row), or with layer, nn::layer_norm with bias nb (may be null).
int mlp_step(smg_mlp *m, const uint16_t *x16, const float *nx, const float *nw, float eps, float *y,
             size_t rows, void *stream, bool layer = false, const float *nb = nullptr) {
    const size_t k = m->up->d.k, d_out = m->down->d.n;
    const bool fused_norm = nx && !layer && rows == 1 && m->gated && k <= 4096 && k % 8 == 0;
    DecodeScratch sc;
    const size_t both = m->gated ? m->up->d.n : 0;
    int rc = decode_scratch(m->device, stream, 0, 0, 0, (nx && !fused_norm ? rows * k : 0) + rows * both +
                                                             rows * d_out,
                            rows * m->hidden, &sc);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    if (nx && !fused_norm) {  // the norm as its own pass (nn::rms_norm / nn::layer_norm)
        if ((e = launch_norm_rows(nx, nw, nb, rows, k, eps, layer, sc.h16, s)) != hipSuccess)
            return fail(SMG_EHIP, layer ? "layer_norm" : "rms_norm", e);
        x16 = sc.h16;
    }
    uint16_t *spare = sc.h16 + (nx && !fused_norm ? rows * k : 0);  // [rows][both], then [rows][d_out]
    if (rows <= 8 && m->gated) {
        BlkArgs b = {};
        b.nx = fused_norm ? nx : nullptr;
        b.nw = nw;
        b.eps = eps;
        b.y = sc.hid;
        b.act = m->act;
        b.nh = (uint32_t)m->hidden;
        if ((e = launch_blk_gemv(m->up->d, rows, x16, b, BS_GLU, fused_norm, s)) != hipSuccess)
            return fail(SMG_EHIP, "gate/up projection", e);
    } else {
        // Mlp::new's up with its activation at the store, or many rows: the
        // GEMM, then (gated) glu over its tiles
        EpArgs ea;
        std::memset(&ea, 0, sizeof(ea));
        if (!m->gated) {
            ea.n_nodes = 1;
            ea.nodes[0].op = EP_OP_ACT;
            ea.nodes[0].aux = m->act;
            ea.fam[0] = ep_family(EP_OP_ACT);
            ea.cls[0] = ep_class(EP_OP_ACT);
        }
        uint16_t *dst = m->gated ? spare : sc.hid;
        const WDev &uw = m->up->d;
        if (m->gated && q4r_supported(uw, rows, 1, (long)uw.k, x16, false) && !q4_gemv_rows(uw, rows, true) &&
            q4r_split_bytes(uw, rows) == 0) {  // one gemm_q4r pass, glu at its store
            if ((e = launch_q4r_glu(uw, rows, sc.hid, m->hidden, x16, m->act, s)) != hipSuccess)
                return fail(SMG_EHIP, "gate/up projection", e);
        } else {
            if ((e = run_q4_dev(m->up->device, uw, rows, dst, x16, ea, false, s)) != hipSuccess)
                return q4_fail("up projection", e);
            if (m->gated && (e = launch_glu(dst, rows, m->hidden, m->act, 1, sc.hid, s)) != hipSuccess)
                return fail(SMG_EHIP, "glu", e);
        }
    }
    if (rows <= 8) {
        BlkArgs r = {};
        r.x = y;
        if ((e = launch_blk_gemv(m->down->d, rows, sc.hid, r, BS_RESID, false, s)) != hipSuccess)
            return fail(SMG_EHIP, "down projection", e);
    } else {
        uint16_t *out16 = spare + rows * both;
        if ((e = q4_add_dev(m->down->device, m->down->d, rows, sc.hid, out16, y, s)) != hipSuccess)
            return q4_fail("down projection", e);
    }
    return SMG_OK;
}

void destroy_attn(smg_attn *a) {
    if (!a) return;
    (void)hipSetDevice(a->device);
    destroy(a->qkv);
    destroy(a->out);
    if (a->rope) (void)hipFree(a->rope);
    for (float *p : a->retired) (void)hipFree(p);
    delete a;
}
void destroy_mlp(smg_mlp *m) {
    if (!m) return;
    destroy(m->up);
    destroy(m->down);
    delete m;
}

// A device-form call hands its pointers straight to the kernels, so each must
// be memory the weights' device can read: that device's own memory, managed
// memory or pinned host memory. Pageable host memory (a malloc'd buffer, a
// numpy array) would make the kernel fault; it is refused with SMG_EINVAL
// instead. The runtime's allocation table answers this on the host (a failed
// lookup's error is cleared so it is not reported by a later call).
bool device_readable(const void *p, int device) {
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (at.type == hipMemoryTypeDevice) return at.device == device;
    return at.type == hipMemoryTypeManaged || at.type == hipMemoryTypeHost;
}

// The pointer query is not a stream operation, so it runs (and refuses a host
// pointer) also while the stream is being captured into a graph: a captured
// call never records a kernel that would read a pageable host address on replay.
int check_dev_ptrs(const char *who, int device, void *stream, const EpPlan &ep,
                   std::initializer_list<const void *> ptrs) {
    (void)who;
    (void)stream;
    for (const void *p : ptrs)
        if (p && !device_readable(p, device))
            return fail(SMG_EINVAL, "device call: an operand pointer is not memory this device can read "
                                    "(host memory must be pinned; device memory must be on the weights' GPU)");
    const EpNode *nodes = ep.nodes();
    for (uint32_t i = 0; i < ep.count(); i++)
        if (nodes[i].ptr && !device_readable(nodes[i].ptr, device))
            return fail(SMG_EINVAL, "device call: an epilogue operand is not memory this device can read "
                                    "(host memory must be pinned; device memory must be on the weights' GPU)");
    return SMG_OK;
}

}  // namespace

int smg::report(int code, const char *what) { return fail(code, what); }

// ============================================================================
extern "C" {

int smg_available(void) {
    pthread_once(&g_avail_once, probe_avail);
    return g_avail;
}

const char *smg_last_error(void) { return g_err.c_str(); }

int smg_ep_check(const ep_desc16 *ep, size_t n) {
    EpPlan p;
    return ep_plan(ep, &p, n);
}

size_t smg_q4_gemv_max_rows(void) { return Q4_GEMV_MAX_ROWS; }

int smg_q4_create(const uint8_t *quants, const uint16_t *scales, const uint16_t *mins, size_t n,
                  size_t k, size_t block, smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_q4(Q4RowMajor{quants, n}, scales, mins, nullptr, nullptr, n, k, block, out);
}

int smg_q4_create_band(const uint8_t *nibbles, const uint16_t *scales, const uint16_t *mins,
                       size_t n, size_t k, size_t block, smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_q4(Q4Band{nibbles, k}, nullptr, nullptr, scales, mins, n, k, block, out);
}

int smg_q2_create(const uint8_t *codes, const uint16_t *scales, const int8_t *codebook, size_t n,
                  size_t k, size_t block, smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_lowbit(W_Q2, Q2RowMajor{codes, n}, scales, false, codebook, n, k, block, out);
}

int smg_q2_create_band(const uint8_t *codes, const uint16_t *scales, const int8_t *codebook,
                       size_t n, size_t k, size_t block, smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_lowbit(W_Q2, Q2Band{codes, round_up(k, 16) * 16}, scales, true, codebook, n, k,
                       block, out);
}

int smg_q1_create(const uint8_t *signs, const uint16_t *scales, int layout, size_t n, size_t k,
                  size_t block, smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_lowbit(W_Q1, Q1RowMajor{signs, n, k, layout}, scales, false, nullptr, n, k, block,
                       out);
}

int smg_q1_create_band(const uint8_t *signs, const uint16_t *scales, size_t n, size_t k,
                       size_t block, smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_lowbit(W_Q1, Q1Band{signs, round_up(k, 16) * 8}, scales, true, nullptr, n, k,
                       block, out);
}

int smg_f16_prepack(const uint16_t *rhs, size_t n, size_t k, long rhs_rs, long rhs_cs,
                    smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_dense(W_F16, rhs, n, k, rhs_rs, rhs_cs, out);
}

int smg_bf16_prepack(const uint16_t *rhs, size_t n, size_t k, long rhs_rs, long rhs_cs,
                     smg_weights **out) {
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    return make_dense(W_BF16, rhs, n, k, rhs_rs, rhs_cs, out);
}

int smg_q4_dequant(const smg_weights *q4, int to_bf16, smg_weights **out) {
    int rc = check_kind(q4, W_Q4);
    if (rc) return rc;
    HIP_TRY(hipSetDevice(q4->device), SMG_EHIP);
    smg_weights *w = new_weights(to_bf16 ? W_BF16 : W_F16, q4->d.n, q4->d.k, 0);
    w->d.k_pad = round_up(q4->d.k_pad, 32);
    WDev src = q4->d;
    src.k_pad = w->d.k_pad;
    void *p;
    if ((rc = alloc_dev(w, w->d.n_pad * w->d.k_pad * 2, &p))) { destroy(w); return rc; }
    w->d.dense = (const uint16_t *)p;
    hipError_t e = launch_q4_dequant_dense(src, (uint16_t *)p, to_bf16 != 0, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) { destroy(w); return fail(SMG_EHIP, "q4 dequant", e); }
    *out = w;
    return SMG_OK;
}

int smg_q4_permute_columns(const smg_weights *q4, const size_t *perm, smg_weights **out) {
    int rc = check_kind(q4, W_Q4);
    if (rc) return rc;
    const size_t n = q4->d.n;
    if ((n && !perm) || !out) return fail(SMG_EINVAL, "null array");
    if (n >= (size_t)1 << 30) return fail(SMG_EINVAL, "too many columns to permute");
    std::vector<int32_t> cols(n);
    for (size_t j = 0; j < n; j++) {
        if (perm[j] >= n) return fail(SMG_EINVAL, "perm entry out of range");
        cols[j] = (int32_t)perm[j];
    }
    return gather_columns(q4, nullptr, cols, out);
}

// GatedLinear's 32-column interleave of two weight sets of one kind
// (src/linear.rs:601-619, lowbit/q1.rs:160-182): 32 of gate, then 32 of up.
static int interleave_kind(int kind, const smg_weights *gate, const smg_weights *up, smg_weights **out) {
    int rc = check_kind(gate, kind);
    if (!rc) rc = check_kind(up, kind);
    if (rc) return rc;
    if (!out) return fail(SMG_EINVAL, "null output");
    const WDev &g = gate->d, &u = up->d;
    if (g.n != u.n || g.k != u.k || g.block != u.block || (g.mins == nullptr) != (u.mins == nullptr))
        return fail(SMG_EINVAL, "gate and up have the same shape and block size");
    if (gate->device != up->device) return fail(SMG_EINVAL, "gate and up are on different devices");
    if (g.n >= (size_t)1 << 29) return fail(SMG_EINVAL, "too many columns to interleave");
    std::vector<int32_t> cols;
    cols.reserve(2 * g.n);
    for (size_t c0 = 0; c0 < g.n; c0 += 32) {
        const size_t c1 = std::min(c0 + 32, g.n);
        for (size_t j = c0; j < c1; j++) cols.push_back((int32_t)j);
        for (size_t j = c0; j < c1; j++) cols.push_back((int32_t)j | (1 << 30));
    }
    return gather_columns(gate, up, cols, out);
}

int smg_q1_interleave(const smg_weights *gate, const smg_weights *up, smg_weights **out) {
    return interleave_kind(W_Q1, gate, up, out);
}

int smg_q4_interleave(const smg_weights *gate, const smg_weights *up, smg_weights **out) {
    return interleave_kind(W_Q4, gate, up, out);
}

void smg_weights_destroy(smg_weights *w) { destroy(w); }

int smg_weights_clone(const smg_weights *w, smg_weights **out) {
    if (!w) return fail(SMG_EINVAL, "null weights");
    HIP_TRY(hipSetDevice(w->device), SMG_EHIP);
    smg_weights *c = new_weights(w->d.kind, w->d.n, w->d.k, w->d.block);
    c->d = w->d;
    struct Field {
        const void *src;
        size_t bytes;
    };
    const size_t code_bytes = cell_grid_rows(w->d.nchunks) * w->d.n_pad * (w->d.kind == W_Q4 ? 16 : 64);
    const size_t sc_bytes = cell_grid_rows(w->d.sc_rows) * w->d.n_pad * 2;
    const size_t dense_bytes = w->d.n_pad * w->d.k_pad * 2;
    const Field f[4] = {{w->d.codes, code_bytes}, {w->d.scales, sc_bytes},
                        {w->d.mins, sc_bytes}, {w->d.dense, dense_bytes}};
    const void **dst[4] = {(const void **)&c->d.codes, (const void **)&c->d.scales,
                           (const void **)&c->d.mins, (const void **)&c->d.dense};
    for (int i = 0; i < 4; i++) {
        if (!f[i].src) continue;
        void *p;
        int rc = alloc_dev(c, f[i].bytes, &p);
        if (rc) { destroy(c); return rc; }
        hipError_t e = hipMemcpy(p, f[i].src, f[i].bytes, hipMemcpyDeviceToDevice);
        if (e != hipSuccess) { destroy(c); return fail(SMG_EHIP, "clone copy", e); }
        *dst[i] = p;
    }
    *out = c;
    return SMG_OK;
}

int smg_weights_info(const smg_weights *w, size_t *n, size_t *k, size_t *block, size_t *bytes) {
    if (!w) return fail(SMG_EINVAL, "null weights");
    if (n) *n = w->d.n;
    if (k) *k = w->d.k;
    if (block) *block = w->d.block;
    if (bytes) *bytes = w->bytes;
    return SMG_OK;
}

int smg_weights_device(const smg_weights *w, int *device) {
    if (!w || !device) return fail(SMG_EINVAL, "null argument");
    *device = w->device;
    return SMG_OK;
}

// ---- host-pointer drop-ins -------------------------------------------------

static int q4_host(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                   const ep_desc16 *ep, bool bf16) {
    int rc = check_kind(w, W_Q4);
    if (rc) return rc;
    const size_t n = w->d.n, k = w->d.k;
    if (m == 0 || n == 0) return SMG_OK;  // q4/matmul.rs:43-44
    const WDev d = w->d;
    const size_t sb = q4_split_bytes(d, m, nullptr, bf16);  // split-K partials in the call's staging
    return host_call(bf16 ? "gemm_gpu_b16b16_q4" : "gemm_gpu_f16f16_q4", w->device, m, n, k, dst,
                     m * n, false, lhs, m * k, ep, sb,
                     [&](uint16_t *dd, const uint16_t *dl, const EpPlan &p, void *sc, hipStream_t s) {
                         const hipError_t e = run_q4(d, m, dd, dl, p.fused, bf16, s, sb ? sc : nullptr, sb);
                         return e == hipSuccess ? plan_tail(p, dd, 1, (long)n, m, n, bf16, s) : e;
                     });
}

int gemm_gpu_f16f16_q4(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep) {
    return q4_host(m, w, dst, lhs, ep, false);
}

int gemm_gpu_b16b16_q4(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep) {
    return q4_host(m, w, dst, lhs, ep, true);
}

static int lowbit_host(int kind, bool mopa, size_t m, const smg_weights *w, uint16_t *dst,
                       const uint16_t *lhs, const ep_desc16 *ep) {
    int rc = check_kind(w, kind);
    if (rc) return rc;
    const size_t n = w->d.n, k = w->d.k;
    if (m == 0 || n == 0) return SMG_OK;  // lowbit/matmul.rs:318-324
    const WDev d = w->d;
    const size_t scratch = mopa ? 0 : lowbit_scratch_bytes(d, m);
    const char *name = mopa ? (kind == W_Q2 ? "gemm_gpu_f16f16_q2" : "gemm_gpu_f16f16_q1")
                            : (kind == W_Q2 ? "gemm_gpu_f16_q2" : "gemm_gpu_f16_q1");
    return host_call(name, w->device, m, n, k, dst, m * n, false, lhs, m * k, ep, scratch,
                     [&](uint16_t *dd, const uint16_t *dl, const EpPlan &p, void *sc, hipStream_t s) {
                         const hipError_t e = mopa ? launch_gemm(d, m, dd, 1, (long)n, dl, 1, (long)k, 1.0f, p.fused,
                                                                 false, s)
                                                   : launch_lowbit_gemv(d, m, dd, dl, p.fused, sc, s);
                         return e == hipSuccess ? plan_tail(p, dd, 1, (long)n, m, n, false, s) : e;
                     });
}

int gemm_gpu_f16_q2(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                    const ep_desc16 *ep) {
    return lowbit_host(W_Q2, false, m, w, dst, lhs, ep);
}
int gemm_gpu_f16_q1(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                    const ep_desc16 *ep) {
    return lowbit_host(W_Q1, false, m, w, dst, lhs, ep);
}
int gemm_gpu_f16f16_q2(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep) {
    return lowbit_host(W_Q2, true, m, w, dst, lhs, ep);
}
int gemm_gpu_f16f16_q1(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep) {
    return lowbit_host(W_Q1, true, m, w, dst, lhs, ep);
}

static int packed_host(bool bf16, size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs,
                       long dst_rs, int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                       const smg_weights *b, uint16_t alpha_bits, uint16_t beta_bits,
                       const ep_desc16 *ep) {
    int rc = check_kind(b, bf16 ? W_BF16 : W_F16);
    if (rc) return rc;
    if (b->d.n != n || b->d.k != k) return fail(SMG_EINVAL, "packed weights shape mismatch");
    if (m == 0 || n == 0) return SMG_OK;
    if (dst_cs <= 0 || dst_rs <= 0 || lhs_cs <= 0 || lhs_rs <= 0)
        return fail(SMG_EINVAL, "strides must be positive");
    const size_t dst_elems = (m - 1) * (size_t)dst_rs + (n - 1) * (size_t)dst_cs + 1;
    const size_t lhs_elems = k ? (m - 1) * (size_t)lhs_rs + (k - 1) * (size_t)lhs_cs + 1 : 0;
    const bool dense_out = (dst_cs == 1 && (size_t)dst_rs == n) || (dst_rs == 1 && (size_t)dst_cs == m);
    const float beta = half_bits_to_float(beta_bits, bf16), alpha = half_bits_to_float(alpha_bits, bf16);
    const WDev d = b->d;
    // a graph past the store's nodes with read_dst: the product goes to the
    // call's scratch, and the graph's pass adds alpha * old C (the store's
    // add_dst step)
    const bool tail_add = read_dst && ep && ep->n_nodes > (uint32_t)EP_FUSED;
    return host_call(bf16 ? "gemm_gpu_b16b16_run_packed" : "gemm_gpu_f16f16_run_packed", b->device,
                     m, n, k, dst, dst_elems, !dense_out || read_dst, lhs, lhs_elems, ep, tail_add ? m * n * 2 : 0,
                     [&](uint16_t *dd, const uint16_t *dl, const EpPlan &p, void *sc, hipStream_t s) {
                         if (tail_add) {
                             uint16_t *prod = (uint16_t *)sc;
                             const hipError_t e = launch_gemm(d, m, prod, 1, (long)n, dl, lhs_cs, lhs_rs, beta,
                                                              p.fused, bf16, s, false, 0.0f);
                             return e == hipSuccess ? launch_ep_tail(prod, (long)n, 1, dd, dst_rs, dst_cs, m, n, alpha,
                                                                     true, p.tail, bf16, s)
                                                    : e;
                         }
                         const hipError_t e = launch_gemm(d, m, dd, dst_cs, dst_rs, dl, lhs_cs, lhs_rs, beta, p.fused,
                                                          bf16, s, read_dst != 0, alpha);
                         return e == hipSuccess ? plan_tail(p, dd, dst_cs, dst_rs, m, n, bf16, s) : e;
                     });
}

int gemm_gpu_f16f16_run_packed(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs,
                               long dst_rs, int read_dst, const uint16_t *lhs, long lhs_cs,
                               long lhs_rs, const smg_weights *b_pack, uint16_t alpha_bits,
                               uint16_t beta_bits, const ep_desc16 *ep) {
    return packed_host(false, m, n, k, dst, dst_cs, dst_rs, read_dst, lhs, lhs_cs, lhs_rs, b_pack,
                       alpha_bits, beta_bits, ep);
}

int gemm_gpu_b16b16_run_packed(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs,
                               long dst_rs, int read_dst, const uint16_t *lhs, long lhs_cs,
                               long lhs_rs, const smg_weights *b_pack, uint16_t alpha_bits,
                               uint16_t beta_bits, const ep_desc16 *ep) {
    return packed_host(true, m, n, k, dst, dst_cs, dst_rs, read_dst, lhs, lhs_cs, lhs_rs, b_pack,
                       alpha_bits, beta_bits, ep);
}

// ---- strided unpacked dense GEMM -------------------------------------------------
// gemm_f16 / gemm_bf16 (src/kernels/f16.rs:126-204, bf16.rs:140-...): B packed
// on the device into the dense layout (a strided gather through LDS), then the
// dense GEMM with A's and C's strides and, under read_dst, alpha * C joined
// before the one rounding. One implementation serves the four reference
// entry points: the f16- and bf16-accumulating ones accumulate in f32 here,
// as the portable path they fall back to does (src/reference.rs:308-387).

// Operand views: A and B may repeat cells (a zero stride broadcasts), C's
// cells must be distinct -- nested strides, one dimension's stride spanning
// the other's whole extent -- since its cells are written in parallel.
static bool read_strides_ok(long rs, long cs) { return rs >= 0 && cs >= 0; }
static bool write_strides_ok(size_t rows, long rs, size_t cols, long cs) {
    if (rs < 0 || cs < 0) return false;
    if (rows > 1 && rs == 0) return false;
    if (cols > 1 && cs == 0) return false;
    return rows <= 1 || cols <= 1 || (size_t)rs >= (size_t)cs * cols || (size_t)cs >= (size_t)rs * rows;
}
static size_t footprint(size_t rows, long rs, size_t cols, long cs) {
    return rows && cols ? (rows - 1) * (size_t)rs + (cols - 1) * (size_t)cs + 1 : 0;
}

static int run_host(bool bf16, const char *name, size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs,
                    long dst_rs, int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs,
                    const uint16_t *rhs, long rhs_cs, long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits) {
    if (m == 0 || n == 0) return SMG_OK;
    if (!dst || (k && (!lhs || !rhs))) return fail(SMG_EINVAL, "null operand");
    if (!write_strides_ok(m, dst_rs, n, dst_cs) || !read_strides_ok(lhs_rs, lhs_cs) ||
        !read_strides_ok(rhs_rs, rhs_cs))
        return fail(SMG_EINVAL, "strides must be non-negative and C's cells distinct");
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    int device = 0;
    HIP_TRY(hipGetDevice(&device), SMG_EHIP);
    WDev d = {};
    d.kind = bf16 ? W_BF16 : W_F16;
    d.n = n;
    d.k = k;
    d.n_pad = round_up(n, 128);
    d.k_pad = round_up(k ? k : 1, 64);
    const size_t rhs_elems = footprint(k, rhs_rs, n, rhs_cs);
    const size_t dense_bytes = round_up(d.n_pad * d.k_pad * 2, 256);
    const size_t dst_elems = footprint(m, dst_rs, n, dst_cs);
    const bool dense_out = (dst_cs == 1 && (size_t)dst_rs == n) || (dst_rs == 1 && (size_t)dst_cs == m);
    const float alpha = half_bits_to_float(alpha_bits, bf16), beta = half_bits_to_float(beta_bits, bf16);
    return host_call(name, device, m, n, k, dst, dst_elems, !dense_out || read_dst, lhs, footprint(m, lhs_rs, k, lhs_cs),
                     nullptr, dense_bytes + rhs_elems * 2,
                     [&](uint16_t *dd, const uint16_t *dl, const EpPlan &p, void *sc, hipStream_t s) {
                         const EpArgs &ea = p.fused;  // no op-graph on these entry points
                         uint16_t *dense = (uint16_t *)sc, *raw = (uint16_t *)((uint8_t *)sc + dense_bytes);
                         if (rhs_elems) {
                             const hipError_t e = hipMemcpyAsync(raw, rhs, rhs_elems * 2, hipMemcpyHostToDevice, s);
                             if (e != hipSuccess) return e;
                         }
                         hipError_t e = launch_pack_dense_strided(raw, rhs_rs, rhs_cs, n, k, d.n_pad, d.k_pad,
                                                                  dense, s);
                         if (e != hipSuccess) return e;
                         WDev w = d;
                         w.dense = dense;
                         return launch_gemm(w, m, dd, dst_cs, dst_rs, dl, lhs_cs, lhs_rs, beta, ea, bf16, s,
                                            read_dst != 0, alpha);
                     });
}

int gemm_gpu_f16f16_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs, int read_dst,
                        const uint16_t *lhs, long lhs_cs, long lhs_rs, const uint16_t *rhs, long rhs_cs,
                        long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits) {
    return run_host(false, "gemm_gpu_f16f16_run", m, n, k, dst, dst_cs, dst_rs, read_dst, lhs, lhs_cs, lhs_rs,
                    rhs, rhs_cs, rhs_rs, alpha_bits, beta_bits);
}
int gemm_gpu_f16f32_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs, int read_dst,
                        const uint16_t *lhs, long lhs_cs, long lhs_rs, const uint16_t *rhs, long rhs_cs,
                        long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits) {
    return run_host(false, "gemm_gpu_f16f32_run", m, n, k, dst, dst_cs, dst_rs, read_dst, lhs, lhs_cs, lhs_rs,
                    rhs, rhs_cs, rhs_rs, alpha_bits, beta_bits);
}
int gemm_gpu_b16b16_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs, int read_dst,
                        const uint16_t *lhs, long lhs_cs, long lhs_rs, const uint16_t *rhs, long rhs_cs,
                        long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits) {
    return run_host(true, "gemm_gpu_b16b16_run", m, n, k, dst, dst_cs, dst_rs, read_dst, lhs, lhs_cs, lhs_rs,
                    rhs, rhs_cs, rhs_rs, alpha_bits, beta_bits);
}
int gemm_gpu_bf16f32_run(size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs, int read_dst,
                         const uint16_t *lhs, long lhs_cs, long lhs_rs, const uint16_t *rhs, long rhs_cs,
                         long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits) {
    return run_host(true, "gemm_gpu_bf16f32_run", m, n, k, dst, dst_cs, dst_rs, read_dst, lhs, lhs_cs, lhs_rs,
                    rhs, rhs_cs, rhs_rs, alpha_bits, beta_bits);
}

int smg_gemm_run_dev(int bf16, size_t m, size_t n, size_t k, uint16_t *dst, long dst_cs, long dst_rs,
                     int read_dst, const uint16_t *lhs, long lhs_cs, long lhs_rs, const uint16_t *rhs,
                     long rhs_cs, long rhs_rs, uint16_t alpha_bits, uint16_t beta_bits, void *stream) {
    if (m == 0 || n == 0) return SMG_OK;
    if (!dst || (k && (!lhs || !rhs))) return fail(SMG_EINVAL, "null operand");
    if (!write_strides_ok(m, dst_rs, n, dst_cs) || !read_strides_ok(lhs_rs, lhs_cs) ||
        !read_strides_ok(rhs_rs, rhs_cs))
        return fail(SMG_EINVAL, "strides must be non-negative and C's cells distinct");
    int device = 0;
    HIP_TRY(hipGetDevice(&device), SMG_EHIP);
    int rc = check_dev_ptrs("smg_gemm_run_dev", device, stream, EpPlan{},
                            {dst, k ? lhs : nullptr, k ? rhs : nullptr});
    if (rc) return rc;
    WDev d = {};
    d.kind = bf16 ? W_BF16 : W_F16;
    d.n = n;
    d.k = k;
    d.n_pad = round_up(n, 128);
    d.k_pad = round_up(k ? k : 1, 64);
    uint16_t *dense = (uint16_t *)dev_pool().get(device, stream, d.n_pad * d.k_pad * 2);
    if (!dense) return fail(SMG_ENOMEM, "smg_gemm_run_dev: scratch hipMalloc");
    hipError_t e = launch_pack_dense_strided(rhs, rhs_rs, rhs_cs, n, k, d.n_pad, d.k_pad, dense,
                                             (hipStream_t)stream);
    if (e == hipSuccess) {
        d.dense = dense;
        EpArgs ea = {};
        const bool b = bf16 != 0;
        e = launch_gemm(d, m, dst, dst_cs, dst_rs, lhs, lhs_cs, lhs_rs, half_bits_to_float(beta_bits, b), ea, b,
                        (hipStream_t)stream, read_dst != 0, half_bits_to_float(alpha_bits, b));
    }
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_gemm_run_dev", e);
}

// The reference's chained link (csrc/gemm_f16f16_q4.h:541-549) with host
// progress words: all of A's depths are awaited first, as its MOPA route does
// (:531-533), then the call runs as gemm_gpu_f16f16_q4 (the same bits, the
// whole op-graph in the kernel) and *done is raised to n once C is stored.
int gemm_gpu_f16f16_q4_chained(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                               const ep_desc16 *ep, size_t *done, const size_t *ready) {
    int rc = check_kind(w, W_Q4);
    if (rc) return rc;
    if (ready && m != 0 && w->d.n != 0)
        while (__atomic_load_n(ready, __ATOMIC_ACQUIRE) < w->d.k) std::this_thread::yield();
    rc = q4_host(m, w, dst, lhs, ep, false);
    if (rc == SMG_OK && done) __atomic_store_n(done, w->d.n, __ATOMIC_RELEASE);
    return rc;
}

int gemm_gpu_f16f16_q4_single(size_t m, size_t n, size_t k) {
    (void)n;
    (void)k;
    return m <= Q4_GEMV_MAX_ROWS ? 1 : 0;
}

// ---- device-pointer entry points -------------------------------------------


int smg_q4_matmul_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                      const ep_desc16 *ep, int bf16, void *stream) {
    int rc = check_kind(w, W_Q4);
    if (rc) return rc;
    if (m == 0 || w->d.n == 0) return SMG_OK;
    EpPlan ep_p;
    if ((rc = ep_plan(ep, &ep_p, w->d.n))) return rc;
    if ((rc = check_dev_ptrs("smg_q4_matmul_dev", w->device, stream, ep_p, {dst, lhs}))) return rc;
    hipError_t e = run_q4_dev(w->device, w->d, m, dst, lhs, ep_p.fused, bf16 != 0, (hipStream_t)stream);
    if (e == hipSuccess) e = plan_tail(ep_p, dst, 1, (long)w->d.n, m, w->d.n, bf16 != 0, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : q4_fail("smg_q4_matmul_dev", e);
}

int smg_q4_chained_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                       const ep_desc16 *ep, unsigned long long *done, const unsigned long long *ready,
                       unsigned int *sync, unsigned int wait_us, void *stream) {
    int rc = check_kind(w, W_Q4);
    if (rc) return rc;
    if (m == 0 || w->d.n == 0) return fail(SMG_EINVAL, "smg_q4_chained_dev: empty call");
    if ((done || ready) && !sync) return fail(SMG_EINVAL, "smg_q4_chained_dev: done / ready need the sync words");
    EpPlan ep_p;
    if ((rc = ep_plan(ep, &ep_p, w->d.n, false))) return rc;
    if ((rc = check_dev_ptrs("smg_q4_chained_dev", w->device, stream, ep_p, {dst, lhs}))) return rc;
    const EpArgs &ea = ep_p.fused;
    // the device wall clock's rate (kHz), read once per device
    static std::atomic<int> clock_khz[64];
    int khz = w->device < 64 ? clock_khz[w->device].load(std::memory_order_relaxed) : 0;
    if (khz <= 0) {
        HIP_TRY(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, w->device), SMG_EHIP);
        if (w->device < 64) clock_khz[w->device].store(khz, std::memory_order_relaxed);
    }
    const unsigned long long us = wait_us ? wait_us : 100000u;
    ChainArgs ch = {ready, done, sync, us * (unsigned long long)(khz > 0 ? khz : 100000) / 1000u, w->d.n};
    hipError_t e = launch_q4_gemv_chained(w->d, m, dst, lhs, ea, ch, (hipStream_t)stream);
    if (e == hipErrorNotSupported)
        return fail(SMG_EINVAL, "smg_q4_chained_dev: needs f16 scale-only Q4, block >= 32, k > 0, m <= 8");
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_q4_chained_dev", e);
}

int smg_lowbit_matmul_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                          const ep_desc16 *ep, void *stream) {
    if (!w) return fail(SMG_EINVAL, "null weights");
    if (w->d.kind != W_Q2 && w->d.kind != W_Q1) return fail(SMG_EKIND, "not low-bit weights");
    if (m == 0 || w->d.n == 0) return SMG_OK;
    EpPlan ep_p;
    int rc = ep_plan(ep, &ep_p, w->d.n);
    if (rc) return rc;
    if ((rc = check_dev_ptrs("smg_lowbit_matmul_dev", w->device, stream, ep_p, {dst, lhs}))) return rc;
    const EpArgs &ea = ep_p.fused;
    const size_t sb = lowbit_scratch_bytes(w->d, m, &ea);
    void *scratch = nullptr;
    if (sb) {
        // several rows (or blocks past one in-kernel pass): the activations
        // are quantized once into a buffer of this stream's own
        scratch = dev_pool().get(w->device, stream, sb);
        if (!scratch) return fail(SMG_ENOMEM, "smg_lowbit_matmul_dev: scratch hipMalloc");
    }
    hipError_t e = launch_lowbit_gemv(w->d, m, dst, lhs, ea, scratch, (hipStream_t)stream);
    if (e == hipSuccess) e = plan_tail(ep_p, dst, 1, (long)w->d.n, m, w->d.n, false, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_lowbit_matmul_dev", e);
}

// As smg_lowbit_matmul_dev, with the quantized activations in the device's
// static `scratch` array (its looked-up address, never the host-side name):
// no device memory is allocated or freed. Nothing there must start at zero:
// the quantization kernel rewrites every entry the product kernel reads.
int smg_lowbit_matmul_dev_noalloc(size_t m, const smg_weights *w, uint16_t *dst,
                                  const uint16_t *lhs, const ep_desc16 *ep, void *stream) {
    if (!w) return fail(SMG_EINVAL, "null weights");
    if (w->d.kind != W_Q2 && w->d.kind != W_Q1) return fail(SMG_EKIND, "not low-bit weights");
    if (m == 0 || w->d.n == 0) return SMG_OK;
    EpPlan ep_p;
    int rc = ep_plan(ep, &ep_p, w->d.n);
    if (rc) return rc;
    if ((rc = check_dev_ptrs("smg_lowbit_matmul_dev_noalloc", w->device, stream, ep_p, {dst, lhs}))) return rc;
    const EpArgs &ea = ep_p.fused;
    const size_t sb = lowbit_scratch_bytes(w->d, m, &ea);
    if (sb > SMG_NOALLOC_SCRATCH_BYTES)
        return fail(SMG_EINVAL, "smg_lowbit_matmul_dev_noalloc: the call needs more scratch than "
                                "SMG_NOALLOC_SCRATCH_BYTES (fewer rows or a shorter K)");
    void *p = nullptr;
    if (sb && (rc = noalloc_scratch(w->device, &p))) return rc;
    hipError_t e = launch_lowbit_gemv(w->d, m, dst, lhs, ea, p, (hipStream_t)stream);
    if (e == hipSuccess) e = plan_tail(ep_p, dst, 1, (long)w->d.n, m, w->d.n, false, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_lowbit_matmul_dev_noalloc", e);
}

int smg_lowbit_mopa_dev(size_t m, const smg_weights *w, uint16_t *dst, const uint16_t *lhs,
                        const ep_desc16 *ep, void *stream) {
    if (!w) return fail(SMG_EINVAL, "null weights");
    if (w->d.kind != W_Q2 && w->d.kind != W_Q1) return fail(SMG_EKIND, "not low-bit weights");
    if (m == 0 || w->d.n == 0) return SMG_OK;
    EpPlan ep_p;
    int rc = ep_plan(ep, &ep_p, w->d.n);
    if (rc) return rc;
    if ((rc = check_dev_ptrs("smg_lowbit_mopa_dev", w->device, stream, ep_p, {dst, lhs}))) return rc;
    const EpArgs &ea = ep_p.fused;
    hipError_t e = launch_gemm(w->d, m, dst, 1, (long)w->d.n, lhs, 1, (long)w->d.k, 1.0f, ea,
                               false, (hipStream_t)stream);
    if (e == hipSuccess) e = plan_tail(ep_p, dst, 1, (long)w->d.n, m, w->d.n, false, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_lowbit_mopa_dev", e);
}

int smg_packed_matmul_dev(size_t m, const smg_weights *b, uint16_t *dst, long dst_cs, long dst_rs,
                          const uint16_t *lhs, long lhs_cs, long lhs_rs, uint16_t beta_bits,
                          const ep_desc16 *ep, int bf16, void *stream) {
    int rc = check_kind(b, bf16 ? W_BF16 : W_F16);
    if (rc) return rc;
    if (m == 0 || b->d.n == 0) return SMG_OK;
    EpPlan ep_p;
    if ((rc = ep_plan(ep, &ep_p, b->d.n))) return rc;
    if ((rc = check_dev_ptrs("smg_packed_matmul_dev", b->device, stream, ep_p, {dst, lhs}))) return rc;
    hipError_t e = launch_gemm(b->d, m, dst, dst_cs, dst_rs, lhs, lhs_cs, lhs_rs,
                               half_bits_to_float(beta_bits, bf16 != 0), ep_p.fused, bf16 != 0,
                               (hipStream_t)stream);
    if (e == hipSuccess) e = plan_tail(ep_p, dst, dst_cs, dst_rs, m, b->d.n, bf16 != 0, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_packed_matmul_dev", e);
}

// ---- decode block ---------------------------------------------------------------

static bool head_shape_ok(size_t heads, size_t kv_heads, size_t hd) {
    return hd % 8 == 0 && hd >= 8 && hd <= 256 && kv_heads > 0 && heads > 0 && heads % kv_heads == 0;
}

int smg_kv_cache_create(size_t heads, size_t kv_heads, size_t head_dim, size_t capacity,
                        smg_kv_cache **out) {
    if (!out) return fail(SMG_EINVAL, "null output");
    if (!head_shape_ok(heads, kv_heads, head_dim))
        return fail(SMG_EINVAL, "head_dim must be a multiple of 8 in 8..=256 and heads a positive multiple of kv_heads");
    if (!smg_available()) return fail(SMG_ENODEV, "no gfx950 device");
    smg_kv_cache *c = new smg_kv_cache();
    (void)hipGetDevice(&c->device);
    c->heads = heads;
    c->kv_heads = kv_heads;
    c->hd = head_dim;
    c->cap = capacity;
    c->len = 0;
    c->scale = 1.0f / std::sqrt((float)head_dim);  // kv_attention.rs:392
    c->k = c->v = nullptr;
    const size_t bytes = std::max<size_t>(capacity * kv_heads * head_dim * 2, 16);
    if (dev_malloc((void **)&c->k, bytes) != hipSuccess || dev_malloc((void **)&c->v, bytes) != hipSuccess ||
        hipMemset(c->k, 0, bytes) != hipSuccess || hipMemset(c->v, 0, bytes) != hipSuccess) {
        smg_kv_cache_destroy(c);
        return fail(SMG_ENOMEM, "KvCache hipMalloc");
    }
    *out = c;
    return SMG_OK;
}

void smg_kv_cache_destroy(smg_kv_cache *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->k) (void)hipFree(c->k);
    if (c->v) (void)hipFree(c->v);
    delete c;
}

int smg_kv_cache_info(const smg_kv_cache *c, size_t *len, size_t *capacity, float *scale) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (len) *len = c->len;
    if (capacity) *capacity = c->cap;
    if (scale) *scale = c->scale;
    return SMG_OK;
}

int smg_kv_cache_truncate(smg_kv_cache *c, size_t len) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    c->len = std::min(c->len, len);
    return SMG_OK;
}

int smg_kv_cache_set_scale(smg_kv_cache *c, float scale) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    c->scale = scale;
    return SMG_OK;
}

int smg_kv_cache_storage(const smg_kv_cache *c, uint16_t **keys, uint16_t **values) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (keys) *keys = c->k;
    if (values) *values = c->v;
    return SMG_OK;
}

int smg_kv_cache_read_dev(const smg_kv_cache *c, uint16_t *keys, uint16_t *values, void *stream) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    const size_t bytes = c->len * c->kv_heads * c->hd * 2;
    if (bytes && keys)
        HIP_TRY(hipMemcpyAsync(keys, c->k, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), SMG_EHIP);
    if (bytes && values)
        HIP_TRY(hipMemcpyAsync(values, c->v, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), SMG_EHIP);
    return SMG_OK;
}

int smg_kv_cache_extend_dev(smg_kv_cache *c, const uint16_t *k, const uint16_t *v, size_t rows,
                            void *stream) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (rows == 0 || !k || !v)
        return fail(SMG_EINVAL, "k and v hold the same whole number of kv_heads * head_dim rows");
    if (c->len + rows > c->cap) return fail(SMG_EINVAL, "KvCache full: the rows do not fit in the cache");
    const size_t ld = c->kv_heads * c->hd;
    HIP_TRY(hipMemcpyAsync(c->k + c->len * ld, k, rows * ld * 2, hipMemcpyDeviceToDevice, (hipStream_t)stream),
            SMG_EHIP);
    HIP_TRY(hipMemcpyAsync(c->v + c->len * ld, v, rows * ld * 2, hipMemcpyDeviceToDevice, (hipStream_t)stream),
            SMG_EHIP);
    c->len += rows;
    return SMG_OK;
}

// rows query rows (f32 [rows][heads hd]), row r attending to keys 0 .. start + r
// (rows = 1, start = len - 1: attention_kv_f16; more rows: the causal form).
static int causal_dev(int device, const float *q, const uint16_t *k, const uint16_t *v, size_t start, size_t rows,
                      size_t heads, size_t kv_heads, size_t hd, float scale, float *out, void *stream) {
    if (!q || !k || !v || !out) return fail(SMG_EINVAL, "null array");
    const size_t qlen = heads * hd;
    uint8_t *bufs[2];
    int rc = carve_scratch(device, stream, 0, {rows * qlen * 2, causal_part_bytes(rows, start + rows, heads, hd)},
                           bufs);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = launch_round_q(q, scale, rows * qlen, (uint16_t *)bufs[0], s);
    if (e == hipSuccess)
        e = causal_attention((uint16_t *)bufs[0], k, v, start, rows, heads, kv_heads, hd, (float *)bufs[1], out,
                             false, s);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "causal attention", e);
}

static int attention_dev(int device, const float *q, const uint16_t *k, const uint16_t *v, size_t len,
                         size_t heads, size_t kv_heads, size_t hd, float scale, float *out, void *stream) {
    if (!head_shape_ok(heads, kv_heads, hd))
        return fail(SMG_EINVAL, "head_dim must be a multiple of 8 in 8..=256 and heads a positive multiple of kv_heads");
    if (len == 0) return fail(SMG_EINVAL, "attention_kv_f16 needs at least one cached key");
    if (!q || !k || !v || !out) return fail(SMG_EINVAL, "null array");
    const size_t qlen = heads * hd, nsplit = attn_splits(len);
    DecodeScratch sc;
    int rc = decode_scratch(device, stream, qlen, nsplit, heads, 0, 0, &sc);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = launch_round_q(q, scale, qlen, sc.q16, s);
    AttnArgs at = {};
    at.q = sc.q16;
    at.k = k;
    at.v = v;
    at.po = sc.po;
    at.pml = sc.pml;
    at.len = (uint32_t)len;
    at.ld = (uint32_t)(kv_heads * hd);
    at.hd = (uint32_t)hd;
    at.heads = (uint32_t)heads;
    at.group = (uint32_t)(heads / kv_heads);
    if (e == hipSuccess) e = launch_attention(at, out, false, s);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "attention", e);
}

int smg_kv_cache_attend_dev(const smg_kv_cache *c, const float *q, float *out, void *stream) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    return attention_dev(c->device, q, c->k, c->v, c->len, c->heads, c->kv_heads, c->hd, c->scale, out, stream);
}

int smg_attention_kv_f16_dev(const float *q, const uint16_t *k, const uint16_t *v, size_t len,
                             size_t heads, size_t kv_heads, size_t head_dim, float scale, float *out,
                             void *stream) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), SMG_EHIP);
    return attention_dev(dev, q, k, v, len, heads, kv_heads, head_dim, scale, out, stream);
}

int smg_attention_kv_causal_f16_dev(const float *q, const uint16_t *k, const uint16_t *v, size_t start,
                                    size_t rows, size_t heads, size_t kv_heads, size_t head_dim, float scale,
                                    float *out, void *stream) {
    if (rows == 0) return fail(SMG_EINVAL, "attention_kv_causal_f16 needs at least one query row");
    if (!head_shape_ok(heads, kv_heads, head_dim))
        return fail(SMG_EINVAL, "head_dim must be a multiple of 8 in 8..=256 and heads a positive multiple of kv_heads");
    if (start > ((size_t)1 << 31) || rows > ((size_t)1 << 31)) return fail(SMG_EINVAL, "start + rows overflows");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), SMG_EHIP);
    return causal_dev(dev, q, k, v, start, rows, heads, kv_heads, head_dim, scale, out, stream);
}

int smg_kv_cache_attend_causal_dev(const smg_kv_cache *c, const float *q, size_t rows, float *out, void *stream) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (rows == 0) return fail(SMG_EINVAL, "attention_kv_causal_f16 needs at least one query row");
    if (rows > c->len) return fail(SMG_EINVAL, "attend_causal: more rows than cached positions");
    return causal_dev(c->device, q, c->k, c->v, c->len - rows, rows, c->heads, c->kv_heads, c->hd, c->scale, out,
                      stream);
}

int smg_rms_norm_f16_dev(const float *x, const float *weight, size_t rows, size_t dim, float eps,
                         uint16_t *y, void *stream) {
    if (dim == 0) return fail(SMG_EINVAL, "a norm needs at least one feature");
    if (rows == 0) return SMG_OK;
    if (!x || !weight || !y) return fail(SMG_EINVAL, "null array");
    hipError_t e = launch_rms_norm(x, weight, rows, dim, eps, y, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "rms_norm", e);
}

int smg_layer_norm_f16_dev(const float *x, const float *weight, const float *bias, size_t rows, size_t dim,
                           float eps, uint16_t *y, void *stream) {
    if (dim == 0) return fail(SMG_EINVAL, "a norm needs at least one feature");
    if (rows == 0) return SMG_OK;
    if (!x || !weight || !y) return fail(SMG_EINVAL, "null array");
    hipError_t e = launch_norm_rows(x, weight, bias, rows, dim, eps, true, y, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "layer_norm", e);
}

int smg_glu_f16_dev(const uint16_t *both, size_t m, size_t n, uint32_t act, uint16_t *y, void *stream) {
    if (act != EP_ACT_SILU && act != EP_ACT_GELU) return fail(SMG_EINVAL, "a gate is silu or gelu");
    if (m == 0 || n == 0) return SMG_OK;
    if (!both || !y) return fail(SMG_EINVAL, "null array");
    hipError_t e = launch_glu(both, m, n, act, 0, y, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "glu", e);
}

int smg_q4_accumulate_dev(size_t m, const smg_weights *w, float *y, const uint16_t *x, void *stream) {
    int rc = check_kind(w, W_Q4);
    if (rc) return rc;
    if (m == 0 || w->d.n == 0) return SMG_OK;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (m <= 8 && !w->d.mins && w->d.block >= (size_t)Q4_CHUNK && w->d.nchunks > 0) {
        BlkArgs r = {};
        r.x = y;
        e = launch_blk_gemv(w->d, m, x, r, BS_RESID, false, s);
    } else {
        DecodeScratch sc;
        if ((rc = decode_scratch(w->device, stream, 0, 0, 0, m * w->d.n, 0, &sc))) return rc;
        e = q4_add_dev(w->device, w->d, m, x, sc.h16, y, s);
    }
    return e == hipSuccess ? SMG_OK : q4_fail("smg_q4_accumulate_dev", e);
}

int smg_attn_create(smg_weights *qkv, smg_weights *out, size_t heads, size_t kv_heads, size_t head_dim,
                    double rope_theta, smg_attn **attn) {
    int rc = check_kind(qkv, W_Q4);
    if (!rc) rc = check_kind(out, W_Q4);
    if (rc) return rc;
    if (!attn) return fail(SMG_EINVAL, "null output");
    if (!head_shape_ok(heads, kv_heads, head_dim) || head_dim % 16 != 0)
        return fail(SMG_EINVAL, "heads must be a positive multiple of kv_heads and head_dim a multiple of 16 up to 256");
    if (qkv->d.n != (heads + 2 * kv_heads) * head_dim)
        return fail(SMG_EINVAL, "qkv has (heads + 2 kv_heads) * head_dim outputs");
    if (out->d.k != heads * head_dim) return fail(SMG_EINVAL, "out takes heads * head_dim inputs");
    if (qkv->d.mins || qkv->d.block < (size_t)Q4_CHUNK || out->d.mins || out->d.block < (size_t)Q4_CHUNK)
        return fail(SMG_EINVAL, "the decode path takes Q4_0 (scale-only) weights with blocks of 32 or more");
    if (qkv->device != out->device) return fail(SMG_EINVAL, "qkv and out are on different devices");
    smg_weights *grouped = nullptr;
    if ((rc = gather_columns(qkv, nullptr, qkv_store_order(qkv->d.n, head_dim), &grouped))) return rc;
    smg_attn *a = new smg_attn();
    a->device = qkv->device;
    a->qkv = grouped;
    a->out = out;
    a->heads = heads;
    a->kv_heads = kv_heads;
    a->hd = head_dim;
    a->theta = rope_theta > 0.0 ? rope_theta : 0.0;
    for (size_t i = 0; i < head_dim / 2; i++)  // model.rs:41-51: (1 / base^(2i/dim)) as f32
        a->inv_freq.push_back((float)(1.0 / std::pow(a->theta, (double)(2 * i) / (double)head_dim)));
    destroy(qkv);  // taken over: its columns now live in `grouped`
    *attn = a;
    return SMG_OK;
}

void smg_attn_destroy(smg_attn *a) { destroy_attn(a); }

int smg_attn_accumulate_dev(smg_attn *a, const uint16_t *x, smg_kv_cache *cache, float *y, size_t m,
                            void *stream) {
    if (!a) return fail(SMG_EINVAL, "null attention");
    if (m == 0) return SMG_OK;
    if (!x || !y) return fail(SMG_EINVAL, "null array");
    if (m > 65535) return fail(SMG_EINVAL, "at most 65535 rows a call");
    if (m > 1) return attn_rows(a, cache, x, y, m, stream);
    return attn_step(a, cache, x, nullptr, nullptr, 0.0f, y, stream);
}

int smg_mlp_create(smg_weights *up, smg_weights *down, uint32_t act, int gated, smg_mlp **mlp) {
    int rc = check_kind(up, W_Q4);
    if (!rc) rc = check_kind(down, W_Q4);
    if (rc) return rc;
    if (!mlp) return fail(SMG_EINVAL, "null output");
    if (act != EP_ACT_SILU && act != EP_ACT_GELU) return fail(SMG_EINVAL, "a gate is silu or gelu");
    const size_t hidden = gated ? up->d.n / 2 : up->d.n;
    if (gated && up->d.n % 2 != 0) return fail(SMG_EINVAL, "a gated up has 2 * hidden outputs");
    if (down->d.k != hidden) return fail(SMG_EINVAL, "down takes up's outputs");
    if (up->device != down->device) return fail(SMG_EINVAL, "up and down are on different devices");
    smg_weights *u = up;
    if (gated) {
        if (up->d.mins || up->d.block < (size_t)Q4_CHUNK)
            return fail(SMG_EINVAL, "a gated MLP takes Q4_0 (scale-only) weights with blocks of 32 or more");
        if ((rc = gather_columns(up, nullptr, glu_store_order(hidden), &u))) return rc;
    }
    smg_mlp *m = new smg_mlp();
    m->device = up->device;
    m->up = u;
    m->down = down;
    m->act = act;
    m->gated = gated != 0;
    m->hidden = hidden;
    if (gated) destroy(up);  // taken over: its columns now live in `u`
    *mlp = m;
    return SMG_OK;
}

void smg_mlp_destroy(smg_mlp *m) { destroy_mlp(m); }

int smg_mlp_accumulate_dev(smg_mlp *m, const uint16_t *x, float *y, size_t rows, void *stream) {
    if (!m) return fail(SMG_EINVAL, "null mlp");
    if (rows == 0) return SMG_OK;
    if (!x || !y) return fail(SMG_EINVAL, "null array");
    return mlp_step(m, x, nullptr, nullptr, 0.0f, y, rows, stream);
}

int smg_block_create_norms(const float *norm1, const float *bias1, float eps1, int layer1, const float *norm2,
                           const float *bias2, float eps2, int layer2, size_t d, smg_attn *attn, smg_mlp *mlp,
                           smg_block **block) {
    if (!attn || !mlp || !block || !norm1 || !norm2) return fail(SMG_EINVAL, "null argument");
    if ((bias1 && !layer1) || (bias2 && !layer2)) return fail(SMG_EINVAL, "only Norm::layer takes a bias");
    if (d == 0 || attn->qkv->d.k != d || attn->out->d.n != d || mlp->up->d.k != d || mlp->down->d.n != d)
        return fail(SMG_EINVAL, "the norms, attention and MLP share the residual's width");
    if (attn->device != mlp->device) return fail(SMG_EINVAL, "attention and MLP are on different devices");
    HIP_TRY(hipSetDevice(attn->device), SMG_EHIP);
    smg_block *b = new smg_block();
    b->device = attn->device;
    b->d = d;
    b->eps1 = eps1;
    b->eps2 = eps2;
    b->layer1 = layer1 != 0;
    b->layer2 = layer2 != 0;
    b->norm1 = b->norm2 = b->bias1 = b->bias2 = nullptr;
    auto upload = [&](float **dst, const float *src) {
        return !src || (dev_malloc((void **)dst, d * 4) == hipSuccess &&
                        hipMemcpy(*dst, src, d * 4, hipMemcpyHostToDevice) == hipSuccess);
    };
    if (!upload(&b->norm1, norm1) || !upload(&b->norm2, norm2) || !upload(&b->bias1, bias1) ||
        !upload(&b->bias2, bias2)) {
        for (float *p : {b->norm1, b->norm2, b->bias1, b->bias2})
            if (p) (void)hipFree(p);
        delete b;
        return fail(SMG_ENOMEM, "block norm weights");
    }
    b->attn = attn;
    b->mlp = mlp;
    *block = b;
    return SMG_OK;
}

int smg_block_create(const float *norm1, float eps1, const float *norm2, float eps2, size_t d,
                     smg_attn *attn, smg_mlp *mlp, smg_block **block) {
    return smg_block_create_norms(norm1, nullptr, eps1, 0, norm2, nullptr, eps2, 0, d, attn, mlp, block);
}

void smg_block_destroy(smg_block *b) {
    if (!b) return;
    (void)hipSetDevice(b->device);
    (void)hipFree(b->norm1);
    (void)hipFree(b->norm2);
    if (b->bias1) (void)hipFree(b->bias1);
    if (b->bias2) (void)hipFree(b->bias2);
    destroy_attn(b->attn);
    destroy_mlp(b->mlp);
    delete b;
}

int smg_block_accumulate_dev(smg_block *b, float *x, smg_kv_cache *cache, size_t rows, void *stream) {
    if (!b) return fail(SMG_EINVAL, "null block");
    if (rows == 0) return SMG_OK;
    if (!x) return fail(SMG_EINVAL, "null array");
    if (rows > 65535) return fail(SMG_EINVAL, "at most 65535 rows a call");
    // x += attn(norm1(x)); x += mlp(norm2(x)) (block.rs:98-105); for one row
    // an RMS norm is fused into the projection that reads it
    const bool fuse = rows == 1 && !b->layer1 && b->d <= 4096 && b->d % 8 == 0;
    int rc;
    if (fuse) {
        rc = attn_step(b->attn, cache, nullptr, x, b->norm1, b->eps1, x, stream);
    } else {
        if ((rc = check_cache(b->attn, cache, rows))) return rc;
        uint8_t *h16;
        if ((rc = carve_scratch(b->device, stream, 0, {rows * b->d * 2}, &h16))) return rc;
        hipError_t e = launch_norm_rows(x, b->norm1, b->bias1, rows, b->d, b->eps1, b->layer1, (uint16_t *)h16,
                                        (hipStream_t)stream);
        if (e != hipSuccess) return fail(SMG_EHIP, b->layer1 ? "layer_norm" : "rms_norm", e);
        // the attention's scratch above the normalized rows
        const size_t base = round_up(rows * b->d * 2, 256);
        rc = rows == 1 ? attn_step(b->attn, cache, (uint16_t *)h16, nullptr, nullptr, 0.0f, x, stream, base)
                       : attn_rows(b->attn, cache, (uint16_t *)h16, x, rows, stream, base);
    }
    if (rc) return rc;
    return mlp_step(b->mlp, nullptr, x, b->norm2, b->eps2, x, rows, stream, b->layer2, b->bias2);
}

// ---- host-slice forms ---------------------------------------------------------------
// Synchronous twins of the device forms above over host arrays, as the
// reference's model parts take them: each returns once its outputs are in
// host memory, and leaves them untouched when it fails.

#define SLICE_BYTES(var, n, elems, width)                                        \
    size_t var;                                                                  \
    if (!slice_bytes((n), (elems), (width), &var)) return fail(SMG_EINVAL, "array size overflows")

int smg_q4_accumulate(size_t m, const smg_weights *w, float *y, const uint16_t *x) {
    int rc = check_kind(w, W_Q4);
    if (rc) return rc;
    if (m == 0 || w->d.n == 0) return SMG_OK;
    if (!x || !y) return fail(SMG_EINVAL, "null array");
    SLICE_BYTES(xb, m, w->d.k, 2);
    SLICE_BYTES(yb, m, w->d.n, 4);
    Slice s[] = {{(void *)x, xb, true, false}, {y, yb, true, true}};
    return slice_call(w->device, s, [&](void **d, void *st) {
        return smg_q4_accumulate_dev(m, w, (float *)d[1], (const uint16_t *)d[0], st);
    });
}

int smg_attn_accumulate(smg_attn *a, const uint16_t *x, smg_kv_cache *cache, float *y, size_t m) {
    if (!a) return fail(SMG_EINVAL, "null attention");
    if (m == 0) return SMG_OK;
    if (!x || !y) return fail(SMG_EINVAL, "null array");
    if (m > 65535) return fail(SMG_EINVAL, "at most 65535 rows a call");
    int rc = check_cache(a, cache, m);
    if (rc) return rc;
    SLICE_BYTES(xb, m, a->qkv->d.k, 2);
    SLICE_BYTES(yb, m, a->out->d.n, 4);
    Slice s[] = {{(void *)x, xb, true, false}, {y, yb, true, true}};
    return slice_call(a->device, s, [&](void **d, void *st) {
        return smg_attn_accumulate_dev(a, (const uint16_t *)d[0], cache, (float *)d[1], m, st);
    });
}

int smg_mlp_accumulate(smg_mlp *m, const uint16_t *x, float *y, size_t rows) {
    if (!m) return fail(SMG_EINVAL, "null mlp");
    if (rows == 0) return SMG_OK;
    if (!x || !y) return fail(SMG_EINVAL, "null array");
    SLICE_BYTES(xb, rows, m->up->d.k, 2);
    SLICE_BYTES(yb, rows, m->down->d.n, 4);
    Slice s[] = {{(void *)x, xb, true, false}, {y, yb, true, true}};
    return slice_call(m->device, s, [&](void **d, void *st) {
        return smg_mlp_accumulate_dev(m, (const uint16_t *)d[0], (float *)d[1], rows, st);
    });
}

int smg_block_accumulate(smg_block *b, float *x, smg_kv_cache *cache, size_t rows) {
    if (!b) return fail(SMG_EINVAL, "null block");
    if (rows == 0) return SMG_OK;
    if (!x) return fail(SMG_EINVAL, "null array");
    if (rows > 65535) return fail(SMG_EINVAL, "at most 65535 rows a call");
    int rc = check_cache(b->attn, cache, rows);
    if (rc) return rc;
    SLICE_BYTES(xb, rows, b->d, 4);
    Slice s[] = {{x, xb, true, true}};
    return slice_call(b->device, s, [&](void **d, void *st) {
        return smg_block_accumulate_dev(b, (float *)d[0], cache, rows, st);
    });
}

int smg_kv_cache_extend(smg_kv_cache *c, const uint16_t *k, const uint16_t *v, size_t rows) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (rows == 0 || !k || !v)
        return fail(SMG_EINVAL, "k and v hold the same whole number of kv_heads * head_dim rows");
    if (rows > c->cap - c->len) return fail(SMG_EINVAL, "KvCache full: the rows do not fit in the cache");
    SLICE_BYTES(kb, rows, c->kv_heads * c->hd, 2);
    Slice s[] = {{(void *)k, kb, true, false}, {(void *)v, kb, true, false}};
    return slice_call(c->device, s, [&](void **d, void *st) {
        return smg_kv_cache_extend_dev(c, (const uint16_t *)d[0], (const uint16_t *)d[1], rows, st);
    });
}

int smg_kv_cache_read(const smg_kv_cache *c, uint16_t *keys, uint16_t *values) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    const size_t bytes = c->len * c->kv_heads * c->hd * 2;
    if (bytes == 0) return SMG_OK;
    Slice s[] = {{keys, bytes, false, true}, {values, bytes, false, true}};
    return slice_call(c->device, s, [&](void **d, void *st) {
        return smg_kv_cache_read_dev(c, (uint16_t *)d[0], (uint16_t *)d[1], st);
    });
}

int smg_kv_cache_attend(const smg_kv_cache *c, const float *q, float *out) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (!q || !out) return fail(SMG_EINVAL, "null array");
    const size_t qb = c->heads * c->hd * 4;
    Slice s[] = {{(void *)q, qb, true, false}, {out, qb, false, true}};
    return slice_call(c->device, s, [&](void **d, void *st) {
        return smg_kv_cache_attend_dev(c, (const float *)d[0], (float *)d[1], st);
    });
}

int smg_kv_cache_attend_causal(const smg_kv_cache *c, const float *q, size_t rows, float *out) {
    if (!c) return fail(SMG_EINVAL, "null cache");
    if (rows == 0) return fail(SMG_EINVAL, "attention_kv_causal_f16 needs at least one query row");
    if (rows > c->len) return fail(SMG_EINVAL, "attend_causal: more rows than cached positions");
    if (!q || !out) return fail(SMG_EINVAL, "null array");
    const size_t qb = rows * c->heads * c->hd * 4;
    Slice s[] = {{(void *)q, qb, true, false}, {out, qb, false, true}};
    return slice_call(c->device, s, [&](void **d, void *st) {
        return smg_kv_cache_attend_causal_dev(c, (const float *)d[0], rows, (float *)d[1], st);
    });
}

int smg_attention_kv_f16(const float *q, const uint16_t *k, const uint16_t *v, size_t len, size_t heads,
                         size_t kv_heads, size_t head_dim, float scale, float *out) {
    if (!head_shape_ok(heads, kv_heads, head_dim))
        return fail(SMG_EINVAL, "head_dim must be a multiple of 8 in 8..=256 and heads a positive multiple of kv_heads");
    if (len == 0) return fail(SMG_EINVAL, "attention_kv_f16 needs at least one cached key");
    if (!q || !k || !v || !out) return fail(SMG_EINVAL, "null array");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), SMG_EHIP);
    SLICE_BYTES(kb, len, kv_heads * head_dim, 2);
    const size_t qb = heads * head_dim * 4;
    Slice s[] = {{(void *)q, qb, true, false}, {(void *)k, kb, true, false}, {(void *)v, kb, true, false},
                 {out, qb, false, true}};
    return slice_call(dev, s, [&](void **d, void *st) {
        return smg_attention_kv_f16_dev((const float *)d[0], (const uint16_t *)d[1], (const uint16_t *)d[2], len,
                                        heads, kv_heads, head_dim, scale, (float *)d[3], st);
    });
}

int smg_attention_kv_causal_f16(const float *q, const uint16_t *k, const uint16_t *v, size_t start, size_t rows,
                                size_t heads, size_t kv_heads, size_t head_dim, float scale, float *out) {
    if (rows == 0) return fail(SMG_EINVAL, "attention_kv_causal_f16 needs at least one query row");
    if (!head_shape_ok(heads, kv_heads, head_dim))
        return fail(SMG_EINVAL, "head_dim must be a multiple of 8 in 8..=256 and heads a positive multiple of kv_heads");
    if (start > ((size_t)1 << 31) || rows > ((size_t)1 << 31)) return fail(SMG_EINVAL, "start + rows overflows");
    if (!q || !k || !v || !out) return fail(SMG_EINVAL, "null array");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), SMG_EHIP);
    SLICE_BYTES(kb, start + rows, kv_heads * head_dim, 2);
    SLICE_BYTES(qb, rows, heads * head_dim, 4);
    Slice s[] = {{(void *)q, qb, true, false}, {(void *)k, kb, true, false}, {(void *)v, kb, true, false},
                 {out, qb, false, true}};
    return slice_call(dev, s, [&](void **d, void *st) {
        return smg_attention_kv_causal_f16_dev((const float *)d[0], (const uint16_t *)d[1], (const uint16_t *)d[2],
                                               start, rows, heads, kv_heads, head_dim, scale, (float *)d[3], st);
    });
}

int smg_rms_norm_f16(const float *x, const float *weight, size_t rows, size_t dim, float eps, uint16_t *y) {
    if (dim == 0) return fail(SMG_EINVAL, "a norm needs at least one feature");
    if (rows == 0) return SMG_OK;
    if (!x || !weight || !y) return fail(SMG_EINVAL, "null array");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), SMG_EHIP);
    SLICE_BYTES(xb, rows, dim, 4);
    Slice s[] = {{(void *)x, xb, true, false}, {(void *)weight, dim * 4, true, false}, {y, xb / 2, false, true}};
    return slice_call(dev, s, [&](void **d, void *st) {
        return smg_rms_norm_f16_dev((const float *)d[0], (const float *)d[1], rows, dim, eps, (uint16_t *)d[2], st);
    });
}

int smg_layer_norm_f16(const float *x, const float *weight, const float *bias, size_t rows, size_t dim, float eps,
                       uint16_t *y) {
    if (dim == 0) return fail(SMG_EINVAL, "a norm needs at least one feature");
    if (rows == 0) return SMG_OK;
    if (!x || !weight || !y) return fail(SMG_EINVAL, "null array");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), SMG_EHIP);
    SLICE_BYTES(xb, rows, dim, 4);
    Slice s[] = {{(void *)x, xb, true, false}, {(void *)weight, dim * 4, true, false},
                 {(void *)bias, bias ? dim * 4 : 0, true, false}, {y, xb / 2, false, true}};
    return slice_call(dev, s, [&](void **d, void *st) {
        return smg_layer_norm_f16_dev((const float *)d[0], (const float *)d[1], (const float *)d[2], rows, dim, eps,
                                      (uint16_t *)d[3], st);
    });
}

#undef SLICE_BYTES

// ---- measurement probes --------------------------------------------------------

int smg_stream_read_dev(const void *p, size_t bytes, void *stream) {
    if (!p || bytes % 16) return fail(SMG_EINVAL, "smg_stream_read_dev: a device pointer and a multiple of 16 bytes");
    hipError_t e = launch_stream_read(p, bytes, nullptr, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_stream_read_dev", e);
}

int smg_stream_read_store_dev(const void *p, size_t bytes, void *out, size_t out_bytes, void *stream) {
    if (!p || bytes % 16 || (out_bytes && !out) || out_bytes % 2)
        return fail(SMG_EINVAL, "smg_stream_read_store_dev: device pointers, bytes a multiple of 16, out_bytes of 2");
    hipError_t e = launch_stream_read_store(p, bytes, (uint16_t *)out, out_bytes / 2, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_stream_read_store_dev", e);
}

int smg_clock_probe_dev(unsigned long long *out, unsigned iters, void *stream) {
    if (!out) return fail(SMG_EINVAL, "null output");
    hipError_t e = launch_clock_probe(out, iters, (hipStream_t)stream);
    return e == hipSuccess ? SMG_OK : fail(SMG_EHIP, "smg_clock_probe_dev", e);
}

}  // extern "C"
