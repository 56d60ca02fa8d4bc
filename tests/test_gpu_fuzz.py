"""Property-based shape fuzz on the GPU (hypothesis, derandomized so every run
draws the same cases): Q4 and Q2/Q1 matmuls at random ragged shapes, block
sizes, forms, output types, epilogue graphs and host or device operands,
against the oracle on the same inputs.

Q4 (src/kernels/q4/matmul.rs:33-102, :187-270): max |g - w| / (1 + |w|) <=
f16_tol(K), 8x that for bf16. Q2 / Q1 on the int8 path
(src/kernels/lowbit/matmul.rs:326-398): identical bits, epilogue included.
Operands are kept small (outputs of order one) so the epilogue's scaling
and subtraction cannot turn a summation-order difference into more than the
bar allows.
"""
import numpy as np
import pytest

from conftest import bf16_tol, f16_tol, max_rel

pytestmark = pytest.mark.gpu

hyp = pytest.importorskip("hypothesis")
st = hyp.strategies
FUZZ = hyp.settings(max_examples=60, deadline=None, derandomize=True, print_blob=True,
                    suppress_health_check=[hyp.HealthCheck.function_scoped_fixture,
                                           hyp.HealthCheck.too_slow, hyp.HealthCheck.data_too_large])

# ragged edges around the tile sizes (16 / 64-column tiles, 32-deep MFMA steps)
DIMS = [1, 2, 15, 16, 17, 31, 33, 63, 64, 65, 97, 127, 129, 200, 257, 300, 513]
ROWS = [1, 2, 3, 4, 5, 7, 8, 9, 16, 33, 64, 65]
# (op, needs an operand of length: "row" m, "col" n, None); op codes as graph.rs
NODE_OPS = [(0, None), (1, None), (11, None), (9, None), (10, None), (2, "row"), (3, "row"),
            (4, "col"), (5, "col"), (13, "col"), (20, "col")]
SCALARS = [0.5, -1.25, 2.0, 0.125, -0.75]   # exact in f16 and bf16
ACTS = [None, 1, 2, 3, 4, 5]                # none, relu, gelu, silu, tanh, sigmoid
ACT_NAMES = {1: "relu", 2: "gelu", 3: "silu", 4: "tanh", 5: "sigmoid"}
EP_METHODS = {0: "add_scalar", 1: "mul_scalar", 11: "sub_scalar", 9: "max", 10: "min",
              2: "add_row", 3: "mul_row", 4: "add_col", 5: "mul_col", 13: "sub_col", 20: "max_col"}


@st.composite
def graphs(draw):
    """A list of (op, scalar index, operand kind) nodes and a trailing act."""
    nodes = draw(st.lists(st.tuples(st.sampled_from(range(len(NODE_OPS))),
                                    st.sampled_from(range(len(SCALARS)))), max_size=3))
    return nodes, draw(st.sampled_from(ACTS))


def _build_ep(smg, nodes, act, m, n, rng, bf16, device):
    """The graph for the library (its operands on the device for a device
    call, host arrays for a host call) and the oracle's node list."""
    cv = _cv(bf16)
    ep, onodes = smg.Epilogue(bf16=bf16), []
    for oi, si in nodes:
        op, operand = NODE_OPS[oi]
        if operand is None:
            v = SCALARS[si]
            ep = getattr(ep, EP_METHODS[op])(v)
            onodes.append((op, 0, v, None, 0))
        else:
            length = m if operand == "row" else n
            lo, hi = (0.5, 1.5) if op in (3, 5) else (-0.5, 0.5)
            vec = cv(rng.uniform(lo, hi, length).astype(np.float32))
            ep = getattr(ep, EP_METHODS[op])(_on_device(vec, bf16) if device else vec)
            onodes.append((op, 0, 0.0, vec, 0))
    if act is not None:
        ep = getattr(ep, ACT_NAMES[act])()
    return ep, onodes


def _cv(bf16):
    import oracle
    return oracle.f32_to_bf16 if bf16 else oracle.f32_to_f16


def _on_device(x, bf16):
    import torch
    return torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16 if bf16 else torch.float16)


def _run(smg, fn, a, w, m, n, ep, device, bf16):
    """fn on host arrays, or on torch tensors of the same bits."""
    if not device:
        c = np.zeros(m * n, np.uint16)
        fn(a, w, c, m, ep)
        return c
    import torch
    dt = torch.bfloat16 if bf16 else torch.float16
    ad = _on_device(a, bf16)
    cd = torch.zeros(m * n, dtype=dt, device="cuda")
    fn(ad, w, cd, m, ep)
    torch.cuda.synchronize()
    return cd.view(torch.int16).cpu().numpy().view(np.uint16)


@FUZZ
@hyp.given(m=st.sampled_from(ROWS), n=st.sampled_from(DIMS), k=st.sampled_from(DIMS),
           block=st.sampled_from([16, 32, 64, 128]), affine=st.booleans(), bf16=st.booleans(),
           device=st.booleans(), graph=graphs(), seed=st.integers(0, 2**31 - 1))
def test_q4_fuzz(smg, orc, m, n, k, block, affine, bf16, device, graph, seed):
    rng = np.random.default_rng(seed)
    nbk = -(-k // block)
    cv = _cv(bf16)
    quants = rng.integers(0, 256, (k * n + 1) // 2, dtype=np.uint8)
    scales = orc.f32_to_f16(rng.uniform(0.002, 0.01, n * nbk).astype(np.float32))
    mins = orc.f32_to_f16(rng.uniform(-0.04, 0.04, n * nbk).astype(np.float32)) if affine else None
    a = cv(rng.uniform(-0.5, 0.5, m * k).astype(np.float32))
    p = smg.Q4Params(block).affine() if affine else smg.Q4Params(block)
    w = smg.Q4Weights.with_params(quants, scales, mins, n, k, p)
    ep, nodes = _build_ep(smg, *graph, m, n, rng, bf16, device)
    fn = smg.matmul_q4_bf16_ep if bf16 else smg.matmul_q4_ep
    got = _run(smg, fn, a, w, m, n, ep, device, bf16)
    want = orc.matmul_q4_ep(a, quants, scales, mins, m, n, k, block, nodes, graph[1], bf16)
    tol = bf16_tol(k) if bf16 else f16_tol(k)
    assert max_rel(got, want, bf16) <= tol, (m, n, k, block, affine, bf16, device, graph)


@FUZZ
@hyp.given(m=st.sampled_from(ROWS), n=st.sampled_from(DIMS), k=st.sampled_from(DIMS),
           block=st.sampled_from([16, 32, 64, 128, 256, 1024]), kind=st.sampled_from([1, 2]),
           inout=st.booleans(), book=st.sampled_from([(-1, 0, 1, 0), (-2, -1, 1, 2), (-128, 127, 3, -7)]),
           device=st.booleans(), graph=graphs(), seed=st.integers(0, 2**31 - 1))
def test_lowbit_fuzz(smg, orc, m, n, k, block, kind, inout, book, device, graph, seed):
    rng = np.random.default_rng(seed)
    nbk = -(-k // block)
    scales = orc.f32_to_f16(rng.uniform(0.0005, 0.004, n * nbk).astype(np.float32))
    a = orc.f32_to_f16(rng.standard_normal(m * k).astype(np.float32))
    if kind == 2:
        codes = rng.integers(0, 256, (k * n + 3) // 4, dtype=np.uint8)
        w = smg.Q2Weights(codes, scales, n, k, smg.Q2Params(block).with_codebook(book))
        fn = smg.matmul_q2_ep
    else:
        codes = rng.integers(0, 256, (k * n + 7) // 8, dtype=np.uint8)
        layout = smg.WeightLayout.InOut if inout else smg.WeightLayout.OutIn
        w = smg.Q1Weights(codes, scales, layout, n, k, block)
        fn = smg.matmul_q1_ep
    ep, nodes = _build_ep(smg, *graph, m, n, rng, False, device)
    got = _run(smg, fn, a, w, m, n, ep, device, False)
    want = orc.matmul_lowbit_ep(kind, a, codes, scales, m, n, k, block, nodes, graph[1],
                                book if kind == 2 else (-1, 0, 1, 0), inout and kind == 1)
    assert np.array_equal(got, want), (m, n, k, block, kind, inout, book, device, graph)
