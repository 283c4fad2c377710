"""The column-blocked path (r > 512: block Gram-Schmidt over 256-column blocks, candidates/kbig.py:69-95, reached
from orth.py:18-19) through the C ABI: bit-identical to the oracle's borth, the robustness gates, strided operands,
hipGraph capture, and the entry points that do not apply to a blocked plan refusing it."""
import ctypes

import pytest
import torch

import oracle
from spanqr_amd import _lib, borth, orth
from spanqr_amd.plan import get_borth_plan, stream_handle
from spanqr_amd.qrbench import gen, metrics

from checks import assert_bits, gate

pytestmark = pytest.mark.gpu

BORTH_CASES = [(1024, 768, "mixed_c4"), (1100, 1024, "rank_half"), (2048, 768, "zero"), (2048, 1024, "huge_1e25"),
               (1536, 1536, "ttf_cu4_t1e-2"), (1000, 768, "dup_cols"), (1280, 1024, "tiny_1e-25"),
               (1088, 1024, "zero_block")]


@pytest.mark.parametrize("K,r,name", BORTH_CASES)
def test_borth_bit_exact(cuda, K, r, name):
    c = next(gen.make_cases(K, r, [name], (0,)))
    print(f"borth {K}x{r} {c.name}", flush=True)
    Q = orth(c.X.to(cuda))
    assert_bits(Q, oracle.borth(c.X.numpy()), f"borth {c.name} {K}x{r}")
    gate(c.X, Q, f"borth {c.name}")


def test_borth_zero_input_nearly_square(cuda):
    """X = 0 with r / K = 0.96: every column is dust completion; block 2 must be completed inside the few directions
    blocks 0-1 leave, and one reorthogonalising projection (kbig.py:91) leaves ~1e-6 there (the oracle's level)"""
    K, r = 800, 768
    X = torch.zeros(K, r)
    print(f"borth zero {K}x{r}", flush=True)
    Q = orth(X.to(cuda))
    assert_bits(Q, oracle.borth(X.numpy()), "borth zero 800x768")
    E = Q.double().T @ Q.double() - torch.eye(r, device=cuda, dtype=torch.float64)
    assert E.abs().max().item() < 2e-6


def test_borth_block_width_and_dispatch(cuda):
    """orth.py:18-20 dispatch and kbig.py:77-78: r <= 256 or not a multiple of 256 is one full-width call"""
    g = torch.Generator().manual_seed(5)
    X = torch.randn(1024, 512, generator=g).to(cuda)
    assert_bits(borth(X), orth(X), "borth at r = 512 is kcholf")
    X = torch.randn(1024, 576, generator=g).to(cuda)            # r > 512, not a multiple of 256: torch.linalg.qr
    Q = orth(X)
    E = Q.double().T @ Q.double() - torch.eye(576, device=cuda, dtype=torch.float64)
    assert E.abs().max().item() < 1e-5
    with pytest.raises(ValueError):                              # b not a multiple of 32: not built natively
        borth(torch.randn(1024, 960, device=cuda), b=80)
    X = torch.randn(1024, 768, generator=g).to(cuda)             # r % b != 0 above 512: full width -> torch.linalg.qr
    Q = borth(X, b=512)
    E = Q.double().T @ Q.double() - torch.eye(768, device=cuda, dtype=torch.float64)
    assert E.abs().max().item() < 1e-5


# borth(X, b, reorth) with the reference's parameters (kbig.py:69): its default b = 512, narrower blocks, and the
# single projection without the reorthogonalisation
OPTION_CASES = [(1024, 1024, 512, True, "mixed_c4"), (1000, 768, 128, True, "rank_half"),
                (1000, 768, 128, False, "mixed_c4"), (1400, 640, 64, True, "zero"), (2048, 1536, 512, False, "dup_cols"),
                (1200, 1024, 256, False, "ttf_cu4_t1e-2"), (1600, 1536, 768, True, "mixed_c4"),
                (2100, 2048, 1024, True, "rank_half"), (1100, 960, 320, False, "mixed_c4"),
                # block widths that are odd multiples of 32: the projection's last 64-wide tile row or column is half
                # used (and every other block starts at an odd multiple of 32)
                (700, 640, 160, True, "mixed_c4"), (600, 576, 96, True, "rank_half"), (400, 256, 32, True, "zero"),
                (1000, 960, 480, True, "mixed_c4"), (900, 864, 288, True, "dup_cols")]


@pytest.mark.parametrize("K,r,b,reorth,name", OPTION_CASES)
def test_borth_block_width_and_reorth_options(cuda, K, r, b, reorth, name):
    c = next(gen.make_cases(K, r, [name], (0,)))
    print(f"borth {K}x{r} b={b} reorth={reorth} {c.name}", flush=True)
    Q = borth(c.X.to(cuda), b=b, reorth=reorth)
    assert_bits(Q, oracle.borth(c.X.numpy(), b, reorth), f"borth b={b} reorth={reorth} {c.name} {K}x{r}")
    if reorth:
        gate(c.X, Q, f"borth b={b} reorth={reorth} {c.name}")
    elif name == "mixed_c4":
        # one projection per block leaves orthogonality at the level of a single Gram-Schmidt pass (2.2e-7 here;
        # 1.1e-5 on the ill-conditioned TTF input, bit-identical to the oracle), and dust completions of dependent
        # columns are not made orthogonal to the earlier blocks (kbig.py:91-92 is what does both), so without
        # reorth: the reference's 1e-6 bar, on a well-conditioned input only
        gate(c.X, Q, f"borth b={b} reorth={reorth} {c.name}", orth_tol=metrics.ORTH_TOL)
    h = get_borth_plan(K, r, b, reorth, cuda)
    assert h.query(_lib.Q_BLOCK_WIDTH) == b and h.query(_lib.Q_BLOCKS) == r // b


def test_borth_large_shape_properties(cuda):
    """eight blocks (r = 2048, the widest TTF layers): repeat bit-identical, the gates hold, and the first block is
    kcholf with its dust slice (checked against the oracle's _kf on s X[:, :256])"""
    K, r = 4096, 2048
    X = gen.bench_input(K, r, seed=3)
    print(f"borth {K}x{r} bench input", flush=True)
    Xd = X.to(cuda)
    Q1 = orth(Xd)
    Q2 = orth(Xd)
    assert_bits(Q1, Q2, "repeat")
    gate(X, Q1, f"borth {K}x{r}")
    Xn = X.numpy()
    s = oracle.pow2_scale(oracle.amax(Xn))
    Z = oracle.dust(K, r)
    Q0 = oracle.orth_dust(Xn[:, :256] * s, Z[:, :256], oracle.gram_rows(K, 256))
    assert_bits(Q1[:, :256], Q0, "first block vs the oracle's _kf")


def test_borth_strided_operands(cuda):
    K, r = 1024, 768
    g = torch.Generator().manual_seed(9)
    X = torch.randn(K, r, generator=g).to(cuda)
    Xw = torch.zeros(K, r + 64, device=cuda)
    Xw[:, :r] = X
    Qw = torch.full((K, r + 128), 7.0, device=cuda)
    plan = get_borth_plan(K, r, 256, True, cuda)   # spanqr_plan_create's plan at r = 768
    print(f"borth strided {K}x{r}", flush=True)
    _lib.check(_lib.lib().spanqr_orth_f32(plan.handle, Xw.data_ptr(), r + 64, Qw.data_ptr(), r + 128, 5e-7, 1e-7, 1e-8,
                                           2, stream_handle(cuda)))
    assert_bits(Qw[:, :r], orth(X), "strided vs contiguous")
    assert (Qw[:, r:] == 7.0).all(), "wrote past the r columns of Q"


def test_borth_graph_capture(cuda):
    K, r = 2048, 1024
    X = gen.bench_input(K, r, seed=4).to(cuda)
    print(f"borth graph {K}x{r}", flush=True)
    Qe = orth(X)
    st = torch.cuda.Stream(cuda)
    st.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(st):
        orth(X)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        Qg = orth(X)
    for rep in range(3):
        gr.replay()
        torch.cuda.synchronize()
        assert_bits(Qg, Qe, f"replay {rep}")
        orth(torch.randn(K, r, device=cuda))          # eager work between replays
        torch.cuda.synchronize()


def test_blocked_plan_refused_where_it_does_not_apply(cuda):
    K, r = 1024, 768
    plan = get_borth_plan(K, r, 256, True, cuda)   # spanqr_plan_create's plan at r = 768
    L = _lib.lib()
    assert L.spanqr_plan_query(plan.handle, _lib.Q_BLOCKS) == 3
    assert L.spanqr_plan_query(plan.handle, _lib.Q_SPLIT_ROWS) == oracle.gram_rows(K, 256)
    X = torch.zeros(K, r, device=cuda)
    ptrs = (ctypes.c_void_p * 1)(X.data_ptr())
    assert L.spanqr_orth_batched_f32(plan.handle, 1, ptrs, r, ptrs, r, 5e-7, 1e-7, 1e-8, 2, stream_handle(cuda)) == -1
    assert b"column-blocked" in L.spanqr_last_error()
    assert L.spanqr_orth_f32(plan.handle, X.data_ptr(), 512, X.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                             stream_handle(cuda)) == -1
