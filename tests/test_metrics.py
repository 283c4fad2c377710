"""The accuracy harness catches what it is meant to catch (restating the reference's own harness self-tests,
tests/test_harness.py:20-130, on the CPU): the generators build what they claim, Householder passes, fp32
Cholesky-QR2 fails where the spec says it does, and planted defects in a Q are reported."""
import pytest
import torch

from spanqr_amd.qrbench import gen, metrics

K, R = 512, 128


def case(name):
    return next(gen.make_cases(K, R, [name], (0,)))


def check(fn, name):
    c = case(name)
    ref = metrics.reference(c.X)
    hres, _ = metrics.run_checked(metrics.householder, c.X, ref)
    res, Q = metrics.run_checked(fn, c.X, ref)
    return res, res.failures(span_ref=hres.span_n), Q


def cholqr2_fp32(X):
    """plain fp32 Cholesky-QR2 (the spec's failing baseline)"""
    Y = X
    for _ in range(2):
        L = torch.linalg.cholesky(Y.T @ Y)
        Y = torch.linalg.solve_triangular(L, Y.T, upper=False).T
    return Y.contiguous()


def test_mixed_singular_values():
    S, _ = metrics.reference(case("mixed_c4").X)
    assert torch.allclose(S, torch.logspace(0, -4, R, dtype=torch.float64), rtol=1e-4)


def test_mixed_is_mixed_on_both_sides():
    n = case("mixed_c6").X.norm(dim=0)
    assert n.max() / n.min() < 10


def test_cases_deterministic():
    a, b = case("ttf_cu4_t1e-2"), case("ttf_cu4_t1e-2")
    assert torch.equal(a.X, b.X) and torch.equal(a.ctx["V"], b.ctx["V"])


def test_ttf_structure():
    c = case("ttf_cu4_t1e-2")
    V = c.ctx["V"].double()
    assert (V.T @ V - torch.eye(R, dtype=torch.float64)).abs().max() < 1e-6
    S, _ = metrics.reference(c.X)
    assert S[0] / S[-1] > 1e5


def test_bench_generator():
    X = gen.ttf_uu(768, 512, seed=0)
    S, _ = metrics.reference(X)
    assert X.shape == (768, 512) and X.dtype == torch.float32
    assert 1e5 < S[0] / S[-1] < 1e9                 # cond(U^T U) up to 1e8, tilted
    assert torch.equal(X, gen.ttf_uu(768, 512, seed=0)) and not torch.equal(X, gen.ttf_uu(768, 512, seed=1))


@pytest.mark.parametrize("name", gen.case_names(K, R))
def test_householder_passes_everything(name):
    res, fails, _ = check(metrics.householder, name)
    assert not [f for f in fails if not (f.startswith("orth") and res.orth <= 2e-6)], fails


@pytest.mark.parametrize("name", ["mixed_c8", "zero", "rank_half", "dup_cols"])
def test_cholqr2_fp32_fails(name):
    _, fails, _ = check(cholqr2_fp32, name)
    assert fails


def test_cholqr2_fp32_fine_when_well_conditioned():
    _, fails, _ = check(cholqr2_fp32, "mixed_c2")
    assert not fails, fails


def _planted(defect):
    return lambda X: defect(torch.linalg.qr(X)[0].contiguous())


def test_detects_zero_column():
    res, fails, _ = check(_planted(lambda Q: torch.cat([Q[:, :-1], torch.zeros_like(Q[:, :1])], 1)), "mixed_c4")
    assert res.bad_cols == 1 and fails


def test_detects_nan():
    res, fails, _ = check(_planted(lambda Q: Q.index_fill(1, torch.tensor([3]), float("nan"))), "mixed_c4")
    assert not res.finite and fails


def test_detects_wrong_span():
    def defect(Q):
        Z = torch.randn(Q.shape[0], 1, generator=torch.Generator().manual_seed(0))
        Z = Z - Q @ (Q.T @ Z)
        Z = Z - Q @ (Q.T @ Z)
        return torch.cat([Q[:, 1:], Z / Z.norm()], 1).contiguous()
    res, fails, _ = check(_planted(defect), "mixed_c4")
    assert res.orth < 1e-6 and res.span_raw > 0.1 and fails


def test_detects_loss_of_orthogonality():
    res, fails, _ = check(_planted(lambda Q: (Q + 1e-5 * Q[:, :1]).contiguous()), "mixed_c4")
    assert res.orth > 1e-6 and fails


def test_detects_nondeterminism():
    state = [0]

    def fn(X):
        state[0] += 1
        Q = torch.linalg.qr(X)[0].contiguous()
        return Q if state[0] % 2 else -Q
    res, fails, _ = check(fn, "mixed_c4")
    assert not res.deterministic and fails


def test_detects_input_modification():
    def fn(X):
        X.mul_(2)
        return torch.linalg.qr(X)[0]
    res, fails, _ = check(fn, "mixed_c4")
    assert not res.input_intact and fails


def test_crash_is_reported():
    def fn(X):
        raise ValueError("boom")
    res, fails, _ = check(fn, "mixed_c4")
    assert res.error and fails


def test_target_gate_is_tighter():
    res, _, _ = check(metrics.householder, "mixed_c4")
    assert metrics.ORTH_TOL_TARGET < metrics.ORTH_TOL
    assert res.failures(orth_tol=1e-30)
