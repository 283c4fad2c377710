"""orth() on the MI355X through the C ABI: the robustness gates of the spec on the adversarial set, the benchmark
inputs, the power-of-2 scale at its rounding edges, strided operands, and hipGraph capture. Every Q is also compared
bit for bit with the CPU oracle on the same input."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from spanqr_amd import _lib, kcholqr_f, orth, stages
from spanqr_amd.plan import get_plan, stream_handle
from spanqr_amd.qrbench import gen, metrics

from checks import assert_bits, gate

pytestmark = pytest.mark.gpu


ADV_SHAPES = [(768, 512), (2048, 512)]
ADV_NAMES = ["cond1e14", "rank1", "right_half_zero", "dup64", "zero", "cond1e8_x1e-25", "cond1e8_x1e25"]


@pytest.fixture(scope="module")
def adversarial_inputs():
    return {(K, r): gen.adversarial(K, r) for K, r in ADV_SHAPES}


@pytest.mark.parametrize("K,r", ADV_SHAPES)
@pytest.mark.parametrize("name", ADV_NAMES)
def test_adversarial(cuda, adversarial_inputs, K, r, name):
    print(f"adversarial {K}x{r} {name}", flush=True)
    X = adversarial_inputs[(K, r)][name]
    Xd = X.to(cuda)
    res, Q = metrics.check_call(orth, Xd, metrics.reference(X))
    assert not res.error, res.error
    assert res.deterministic and res.input_intact and res.sync_free
    assert stages.scalars(K, r, cuda)[7].item() == 0, "grid barrier timed out"
    gate(X, Q, name)
    assert_bits(Q, oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows), "Q vs oracle")


# the benchmark inputs: the headline shapes (768x512; 17408x256 with N = 5120), both seeds of the 0.8B layer shapes
# (1024, 2048, 3584 x 256, N = K), the other 27B shapes (N = 5120) and 2048x512
@pytest.mark.parametrize("K,r,seed", [(1024, 256, 0), (1024, 256, 1), (2048, 256, 0), (2048, 256, 1),
                                      (3584, 256, 0), (3584, 256, 1), (5120, 256, 0), (6144, 256, 0),
                                      (17408, 256, 0), (768, 512, 0), (2048, 512, 0)])
def test_benchmark_inputs(cuda, K, r, seed):
    print(f"bench input {K}x{r} seed {seed}", flush=True)
    X = gen.bench_input(K, r, seed=seed)
    Q = orth(X.to(cuda))
    gate(X, Q, f"{K}x{r} seed {seed}")
    assert_bits(Q, oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows), "Q vs oracle")


def test_lds_limit_shared_by_plans(cuda):
    """a kernel's dynamic-LDS limit is shared by every plan that launches it: a plan made later with a smaller need
    (16400 x 320 runs the same two-row-block solve as 16400 x 512 with less LDS) must not lower it under the first"""
    K, r = 16400, 512
    X = gen.bench_input(K, r, seed=2)
    Xd = X.to(cuda)
    Q0 = kcholqr_f(Xd)
    get_plan(K, 320, cuda)
    kcholqr_f(torch.randn(K, 320, device=cuda))
    print("lds limit: 16400x512 after a 16400x320 plan", flush=True)
    Q1 = kcholqr_f(Xd)
    assert_bits(Q1, Q0, "16400x512 after a 16400x320 plan vs before")
    assert_bits(Q1, oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows), "Q vs oracle")


def _tie_band_values():
    """max|x| values at the edges of round(log2): mantissas around sqrt(2) at small, middle and large exponents,
    where fp32 log2 lands exactly on e + 1/2 and round-half-even decides"""
    out = []
    for e in (-120, -63, -2, -1, 0, 1, 2, 3, 41, 100, 126):
        for mb in (0x3504C0, 0x3504F3, 0x3504F4, 0x3504F8, 0x350510):
            out.append(float(np.array([((e + 127) << 23) | mb], np.uint32).view(np.float32)[0]))
    return out


def test_pow2_scale_edges(cuda):
    K, r = 256, 64
    rng = np.random.default_rng(0)
    base = (0.5 * rng.uniform(-1, 1, (K, r))).astype(np.float32)
    for m in _tie_band_values():
        X = (base * np.float32(m)).astype(np.float32)
        X[3, 5] = np.float32(m)
        Q = orth(torch.from_numpy(X).to(cuda))
        s = stages.scalars(K, r, cuda)[0].item()
        assert np.float32(s) == oracle.pow2_scale(np.float32(m)), f"max {m!r}: scale {s} vs {oracle.pow2_scale(m)}"
        assert_bits(Q, oracle.orth(X, get_plan(K, r, cuda).split_rows), f"Q at max {m!r}")


@pytest.mark.parametrize("where", ["first", "last", "middle", "strided"])
def test_scale_of_tall_x(cuda, where):
    """X of 2^20 elements and more (the amax's 1024-thread workgroups): the maximum is found wherever it sits, and a
    row stride wider than r hides the columns past r (filled with 1e30 here)"""
    K, r = 8192, 128
    rng = np.random.default_rng(1)
    X = rng.uniform(-1, 1, (K, r)).astype(np.float32)
    i, j = {"first": (0, 0), "last": (K - 1, r - 1), "middle": (4099, 77), "strided": (K - 1, r - 1)}[where]
    X[i, j] = np.float32(-3.0e4)
    print(f"scale of {K}x{r}, maximum at {where}", flush=True)
    plan = get_plan(K, r, cuda)
    pad = 4 if where == "strided" else 0
    Xp = torch.full((K, r + pad), 1e30, device=cuda)
    Xp[:, :r] = torch.from_numpy(X).to(cuda)
    Q = torch.empty(K, r, device=cuda)
    _lib.check(_lib.lib().spanqr_orth_f32(plan.handle, Xp.data_ptr(), r + pad, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                                          stream_handle(cuda)))
    torch.cuda.synchronize()
    s = stages.scalars(K, r, cuda)[0].item()
    assert np.float32(s) == oracle.pow2_scale(np.float32(3.0e4)) == np.float32(2.0 ** -15), f"scale {s}"


def test_strided_operands(cuda):
    """ldx > r and ldq > r through the C ABI (the reference copies to contiguous first, kcholqr.py:100)"""
    K, r, pad = 1024, 256, 12
    X = next(gen.make_cases(K, r, ["mixed_c6"], (0,))).X
    Xp = torch.full((K, r + pad), float("nan"), device=cuda)
    Xp[:, :r] = X.to(cuda)
    Qp = torch.full((K, r + pad), -7.0, device=cuda)
    plan = get_plan(K, r, cuda)
    _lib.check(_lib.lib().spanqr_orth_f32(plan.handle, Xp.data_ptr(), r + pad, Qp.data_ptr(), r + pad, 5e-7, 1e-7,
                                          1e-8, 2, stream_handle(cuda)))
    torch.cuda.synchronize()
    assert torch.all(Qp[:, r:] == -7.0), "wrote outside Q's columns"
    assert_bits(Qp[:, :r].contiguous(), kcholqr_f(X.to(cuda)), "strided vs contiguous")


def test_abi_rejects_bad_operands(cuda):
    K, r = 256, 64
    plan = get_plan(K, r, cuda)
    X = torch.zeros(K, r + 1, device=cuda)
    Q = torch.zeros(K, r, device=cuda)
    f = _lib.lib().spanqr_orth_f32
    st = stream_handle(cuda)
    assert f(plan.handle, X.data_ptr(), r + 1, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2, st) == -1   # ld % 4
    assert f(plan.handle, X.data_ptr() + 4, r, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2, st) == -1   # alignment
    assert f(plan.handle, None, r, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2, st) == -1
    assert f(plan.handle, X.data_ptr(), r, Q.data_ptr(), r - 4, 5e-7, 1e-7, 1e-8, 2, st) == -1   # ldq < r
    assert f(plan.handle, X.data_ptr(), 1 << 24, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2, st) == -1  # ldx >= 2^24
    assert _lib.lib().spanqr_last_error()


@pytest.mark.parametrize("K,r", [(2048, 256), (768, 512), (17408, 256)])
def test_graph_capture_replays(cuda, K, r):
    """the whole call captured into one hipGraph; replays with eager work in between equal the eager result (both
    Newton-Schulz apply forms: two-buffer at 2048x256 and 768x512, D in registers at 17408x256)"""
    X = gen.bench_input(K, r, seed=1).to(cuda)
    Qe = kcholqr_f(X)
    st = torch.cuda.Stream(cuda)
    st.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(st):
        kcholqr_f(X)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        Qg = kcholqr_f(X)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert_bits(Qg, Qe, f"replay {i}")
        kcholqr_f(torch.randn(K, r, device=cuda))    # eager work on another plan's stream between replays
        torch.cuda.synchronize()


def test_keyword_arguments(cuda):
    """eps, alpha, tau and ns reach the kernels as the reference's keywords (kcholqr.py:92)"""
    K, r = 512, 128
    X = next(gen.make_cases(K, r, ["mixed_c8"], (0,))).X
    KS = get_plan(K, r, cuda).split_rows
    for kw in (dict(eps=1e-6), dict(alpha=1e-6), dict(tau=1e-7), dict(ns=1), dict(ns=0), dict(ns=3)):
        Q = kcholqr_f(X.to(cuda), **kw)
        assert_bits(Q, oracle.orth(X.numpy(), KS, **kw), f"kcholqr_f({kw})")


@pytest.mark.parametrize("K,r", [(768, 512), (2048, 512), (1024, 256), (3584, 256), (6144, 256), (17408, 256)])
def test_solve_runs_in_the_cholesky_launch(cuda, K, r):
    """at the benchmark shapes each pass's solve runs in its Cholesky's launch, and the call stays bit-exact"""
    plan = get_plan(K, r, cuda)
    assert plan.solve_rows > 0, f"{K}x{r}: the solve is a separate launch"
    X = gen.bench_input(K, r, seed=3)
    print(f"fused solve {K}x{r}: {plan.solve_rows} rows per solve workgroup", flush=True)
    assert_bits(kcholqr_f(X.to(cuda)), oracle.orth(X.numpy(), plan.split_rows), f"{K}x{r} vs oracle")


@pytest.mark.parametrize("K,r", [(5000, 64), (4500, 128), (4111, 192), (4100, 256), (9217, 256)])
def test_tall_solve_in_cholesky_launch(cuda, K, r):
    """X taller than one row block per CU: the solve in the Cholesky's launch runs one wavefront per 16 rows, 2 to 8
    of them per workgroup (as many workgroups as CUs are free), at every column-block count (r/32 = 2, 4, 6, 8), with a
    ragged last row block and a last workgroup with fewer row blocks than the others"""
    plan = get_plan(K, r, cuda)
    assert 32 <= plan.solve_rows <= 128, f"{K}x{r}: expected the wavefront-per-row-block solve, got {plan.solve_rows}"
    g = torch.Generator().manual_seed(K + r)
    X = torch.randn(K, r, generator=g) * torch.logspace(0, -3, r)
    print(f"tall solve {K}x{r}", flush=True)
    Q = kcholqr_f(X.to(cuda))
    assert_bits(Q, oracle.orth(X.numpy(), plan.split_rows), f"{K}x{r} vs oracle")
    gate(X, Q, f"{K}x{r}")


@pytest.mark.parametrize("K,r", [(1100, 544), (3000, 736), (2048, 992)])
def test_full_width_above_512_columns(cuda, K, r):
    """orth.py:20: above 512 columns, r not a multiple of 256 runs kcholf at full width -- bit-exact vs the oracle,
    within the gates, and the same through the C ABI's orth-dispatch plan (spanqr_plan_create)"""
    X = next(gen.make_cases(K, r, ["mixed_c6"], (0,))).X
    plan = get_plan(K, r, cuda)
    assert plan.query(_lib.Q_BLOCKS) == 0
    print(f"full width {K}x{r}: {plan.chol_grid} Cholesky workgroups", flush=True)
    Q = orth(X.to(cuda))
    assert_bits(Q, oracle.orth(X.numpy(), plan.split_rows), f"{K}x{r} vs oracle")
    gate(X, Q, f"{K}x{r}")
    h = ctypes.c_void_p()
    _lib.check(_lib.lib().spanqr_plan_create(K, r, cuda.index or 0, ctypes.byref(h)))
    try:
        assert _lib.lib().spanqr_plan_query(h, _lib.Q_BLOCKS) == 0
        Xd, Qd = X.to(cuda), torch.empty(K, r, device=cuda)
        _lib.check(_lib.lib().spanqr_orth_f32(h, Xd.data_ptr(), r, Qd.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                                              stream_handle(cuda)))
        torch.cuda.synchronize()
        assert_bits(Qd, Q, "spanqr_plan_create's plan vs orth")
    finally:
        _lib.lib().spanqr_plan_destroy(h)


def test_kcholf_full_width_where_orth_is_blocked(cuda):
    """at r = 768 orth takes borth over 256-column blocks (orth.py:18-19) while kcholqr_f runs at full width, as the
    reference's kcholqr_f does (kcholqr.py:92-112)"""
    K, r = 1100, 768
    X = next(gen.make_cases(K, r, ["mixed_c4"], (1,))).X
    print(f"kcholf full width {K}x{r}", flush=True)
    Qk = kcholqr_f(X.to(cuda))
    assert_bits(Qk, oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows), "kcholqr_f vs oracle")
    assert_bits(orth(X.to(cuda)), oracle.borth(X.numpy()), "orth (borth) vs oracle")


@pytest.mark.parametrize("K,r", [(3000, 736), (1100, 1024), (2048, 512)])
def test_repeated_calls_bit_identical(cuda, K, r):
    """forty calls on one plan give the same bits: every flag and column credit is published only after the L2
    write-back of what it covers has completed (a flag that overtook the write-back let readers on another XCD see
    the previous launch's values, most often at these shapes)"""
    X = next(gen.make_cases(K, r, ["mixed_c6"], (0,))).X.to(cuda)
    print(f"repeated calls {K}x{r}", flush=True)
    Q0 = kcholqr_f(X)
    for i in range(40):
        assert_bits(kcholqr_f(X), Q0, f"call {i + 1}")
