"""Batched orth through the C ABI (spanqr_orth_batched_f32, orth_many): every Q of a batch is bit-identical to the
single call on that X, also when the Cholesky runs in several launches, when shape groups are mixed with shapes
outside the native kernels, and under hipGraph capture."""
import ctypes

import pytest
import torch

import oracle
from spanqr_amd import _lib, kcholqr_f, kcholqr_f_many, orth, orth_many
from spanqr_amd.plan import get_plan, stream_handle
from spanqr_amd.qrbench import gen

from checks import assert_bits, gate

pytestmark = pytest.mark.gpu


def test_batch_matches_single_calls(cuda):
    K, r, n = 1024, 256, 5
    Xs = [gen.bench_input(K, r, seed=s) for s in range(n)]
    print(f"batched {n} x {K}x{r}", flush=True)
    Qs = kcholqr_f_many([X.to(cuda) for X in Xs])
    for i, (X, Q) in enumerate(zip(Xs, Qs)):
        assert_bits(Q, kcholqr_f(X.to(cuda)), f"batch element {i} vs single call")
    gate(Xs[3], Qs[3], "batch element 3")
    assert_bits(Qs[2], oracle.orth(Xs[2].numpy(), get_plan(K, r, cuda).split_rows), "batch element 2 vs oracle")


def test_full_width_batch_matches_single_calls(cuda):
    """kcholf at full width above 512 columns (tile rows split over several owner workgroups), batched: each Q equals
    the single call and the oracle"""
    K, r, n = 700, 544, 3
    g = torch.Generator().manual_seed(11)
    Xs = [torch.randn(K, r, generator=g) * torch.logspace(0, -4, r) for _ in range(n)]
    print(f"batched {n} x {K}x{r}", flush=True)
    Qs = kcholqr_f_many([X.to(cuda) for X in Xs])
    for i, (X, Q) in enumerate(zip(Xs, Qs)):
        assert_bits(Q, kcholqr_f(X.to(cuda)), f"batch element {i} vs single call")
    assert_bits(Qs[1], oracle.orth(Xs[1].numpy(), get_plan(K, r, cuda).split_rows), "batch element 1 vs oracle")
    gate(Xs[1], Qs[1], "batch element 1")


def test_cholesky_in_several_launches(cuda):
    """more matrices than one Cholesky launch holds (every workgroup of a launch must be resident at once)"""
    K, r, n = 512, 512, 24
    plan = get_plan(K, r, cuda, n)
    print(f"batched {n} x {K}x{r}, {plan.chol_batch} per Cholesky launch", flush=True)
    if plan.chol_batch >= n:
        pytest.skip(f"the device holds all {n} Cholesky factorisations in one launch")
    g = torch.Generator().manual_seed(7)
    Xs = [torch.randn(K, r, generator=g) for _ in range(n)]
    Qs = kcholqr_f_many([X.to(cuda) for X in Xs])
    for i in (0, plan.chol_batch - 1, plan.chol_batch, n - 1):
        assert_bits(Qs[i], kcholqr_f(Xs[i].to(cuda)), f"batch element {i} vs single call")
    assert_bits(Qs[n - 1], oracle.orth(Xs[n - 1].numpy(), plan.split_rows), "last element vs oracle")


def test_orth_many_groups_shapes_and_keeps_order(cuda):
    g = torch.Generator().manual_seed(3)
    shapes = [(1024, 256), (768, 512), (1024, 256), (1000, 96), (768, 512), (1024, 256), (300, 64), (500, 80),
              (1000, 96)]
    Xs = [torch.randn(K, r, generator=g).to(cuda) for K, r in shapes]
    Xs[2] = Xs[2] * 1e-20                                   # a scale edge inside a group
    Qs = orth_many(Xs)
    assert len(Qs) == len(Xs)
    for i, (X, Q) in enumerate(zip(Xs, Qs)):
        assert Q.shape == X.shape
        if X.shape[1] % 32:     # outside the native kernels: torch.linalg.qr, as the reference (kcholqr.py:98-99)
            E = Q.T.double() @ Q.double() - torch.eye(X.shape[1], device=cuda, dtype=torch.float64)
            assert E.abs().max().item() < 1e-5, f"orth_many[{i}] fallback not orthonormal"
        else:
            assert_bits(Q, orth(X), f"orth_many[{i}] vs orth ({tuple(X.shape)})")


def test_batched_call_under_graph_capture(cuda):
    K, r, n = 2048, 256, 3
    Xs = [gen.bench_input(K, r, seed=10 + s).to(cuda) for s in range(n)]
    Qe = kcholqr_f_many(Xs)
    st = torch.cuda.Stream(cuda)
    st.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(st):
        kcholqr_f_many(Xs)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        Qg = kcholqr_f_many(Xs)
    for rep in range(3):
        gr.replay()
        torch.cuda.synchronize()
        for i in range(n):
            assert_bits(Qg[i], Qe[i], f"replay {rep} element {i}")
        kcholqr_f_many([torch.randn(K, r, device=cuda) for _ in range(n)])   # eager work between replays
        torch.cuda.synchronize()


def test_batched_abi_rejects_bad_operands(cuda):
    K, r = 256, 64
    plan = get_plan(K, r, cuda, 2)
    X = torch.zeros(2, K, r, device=cuda)
    Q = torch.zeros(2, K, r, device=cuda)
    f = _lib.lib().spanqr_orth_batched_f32
    st = stream_handle(cuda)

    def arr(*ptrs):
        return (ctypes.c_void_p * len(ptrs))(*ptrs)

    good_x, good_q = arr(X[0].data_ptr(), X[1].data_ptr()), arr(Q[0].data_ptr(), Q[1].data_ptr())
    assert f(plan.handle, 3, good_x, r, good_q, r, 5e-7, 1e-7, 1e-8, 2, st) == -1          # n > batch
    assert f(plan.handle, 0, good_x, r, good_q, r, 5e-7, 1e-7, 1e-8, 2, st) == -1
    assert f(plan.handle, 2, arr(X[0].data_ptr(), X[1].data_ptr() + 4), r, good_q, r, 5e-7, 1e-7, 1e-8, 2, st) == -1
    assert b"X[1]" in _lib.lib().spanqr_last_error()
    assert f(plan.handle, 2, good_x, r, arr(Q[0].data_ptr(), None), r, 5e-7, 1e-7, 1e-8, 2, st) == -1
    assert b"Q[1]" in _lib.lib().spanqr_last_error()
    assert f(plan.handle, 2, None, r, good_q, r, 5e-7, 1e-7, 1e-8, 2, st) == -1
    assert f(plan.handle, 2, good_x, r, good_q, r, 5e-7, 1e-7, 1e-8, 2, st) == 0


def test_batched_layer_set(cuda):
    """the batched layer set of one training step: 12 layers at 768x512 and 12 at 2048x512 (attention and down_proj
    of the 110M model), independent cond-1e8 inputs (seeds 100 + 12 g + i), through orth_many: every Q bit-identical
    to its single call and to the oracle, and through the spec's gates"""
    groups = [(768, 512, 12), (2048, 512, 12)]
    Xs = [gen.ttf_uu(K, r, N=K, seed=100 + 12 * gi + i) for gi, (K, r, n) in enumerate(groups) for i in range(n)]
    print(f"batched layer set: {[f'{n} x {K}x{r}' for K, r, n in groups]}", flush=True)
    Qs = orth_many([X.to(cuda) for X in Xs])
    for i, (X, Q) in enumerate(zip(Xs, Qs)):
        K, r = X.shape
        Qo = oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows)
        assert_bits(Q, Qo, f"layer {i} ({K}x{r}), batched, vs oracle")
        assert_bits(orth(X.to(cuda)), Qo, f"layer {i} ({K}x{r}), single call, vs oracle")
        gate(X, Q, f"layer {i} ({K}x{r})")


def test_batched_tall_solve(cuda):
    """a batch whose solves run one wavefront per 16 rows in the Cholesky's launches"""
    K, r, n = 5000, 128, 3
    g = torch.Generator().manual_seed(9)
    Xs = [torch.randn(K, r, generator=g) for _ in range(n)]
    print(f"batched {n} x {K}x{r}", flush=True)
    Qs = kcholqr_f_many([X.to(cuda) for X in Xs])
    for i in range(n):
        assert_bits(Qs[i], oracle.orth(Xs[i].numpy(), get_plan(K, r, cuda, n).split_rows), f"element {i} vs oracle")


def test_batched_ns_apply_forms_agree(cuda):
    """12 x 1100x192: the batch's Newton-Schulz apply keeps D's columns in registers (eight row groups per matrix),
    each single call uses the two-buffer form; every Q is bit-identical across the two"""
    K, r, n = 1100, 192, 12
    g = torch.Generator().manual_seed(13)
    Xs = [torch.randn(K, r, generator=g) * torch.logspace(0, -3, r) for _ in range(n)]
    print(f"batched {n} x {K}x{r}", flush=True)
    Qs = kcholqr_f_many([X.to(cuda) for X in Xs])
    for i in (0, 5, n - 1):
        assert_bits(Qs[i], kcholqr_f(Xs[i].to(cuda)), f"batch element {i} vs single call")
    assert_bits(Qs[n - 1], oracle.orth(Xs[n - 1].numpy(), get_plan(K, r, cuda).split_rows), "last element vs oracle")


def test_batched_long_splits(cuda):
    """3 x 8192x384: 352-row Gram splits, so every matrix's plain Grams go through the register-operand kernel in
    one launch per pass; each Q bit-identical to its single call, one to the oracle"""
    K, r, n = 8192, 384, 3
    plan = get_plan(K, r, cuda, n)
    assert plan.split_rows >= 320
    g = torch.Generator().manual_seed(17)
    Xs = [torch.randn(K, r, generator=g) * torch.logspace(0, -4, r) for _ in range(n)]
    print(f"batched {n} x {K}x{r}", flush=True)
    Qs = kcholqr_f_many([X.to(cuda) for X in Xs])
    for i in range(n):
        assert_bits(Qs[i], kcholqr_f(Xs[i].to(cuda)), f"batch element {i} vs single call")
    assert_bits(Qs[1], oracle.orth(Xs[1].numpy(), plan.split_rows), "element 1 vs oracle")
