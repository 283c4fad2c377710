"""The Cholesky's failure path through the C ABI: when one of its bounded waits gives up (forced here from the host by
a spin limit of zero, so every kernel still ends normally), the call's Q comes out NaN and the wait-error word is set;
the next normal call clears the word and is bit-identical to the oracle again. The waits need every workgroup of a
launch resident at once; a give-up is how a violation shows (the reference's cooperative launch fails instead)."""
import numpy as np
import pytest
import torch

import oracle
from spanqr_amd import _lib, kcholqr_f, kcholqr_f_many, stages
from spanqr_amd.plan import get_plan
from spanqr_amd.qrbench import gen

from checks import assert_bits

pytestmark = pytest.mark.gpu

DEFAULT_LIMIT = 1 << 20


@pytest.fixture
def zero_spin_limit():
    _lib.lib().spanqr_debug_spin_limit(0)
    try:
        yield
    finally:
        _lib.lib().spanqr_debug_spin_limit(DEFAULT_LIMIT)


def test_wait_give_up_makes_q_nan_and_is_cleared(cuda):
    K, r = 768, 512
    X = gen.ttf_uu(K, r, N=K, seed=0)
    Xd = X.to(cuda)
    Q0 = kcholqr_f(Xd)
    torch.cuda.synchronize()
    assert stages.scalars(K, r, cuda)[7].item() == 0.0
    print("failure path: spin limit 0 at 768x512", flush=True)
    _lib.lib().spanqr_debug_spin_limit(0)
    try:
        Qf = kcholqr_f(Xd)
        torch.cuda.synchronize()
    finally:
        _lib.lib().spanqr_debug_spin_limit(DEFAULT_LIMIT)
    err = stages.scalars(K, r, cuda)[7].view(torch.int32).item()
    assert err != 0, "no wait gave up with a spin limit of 0"
    assert torch.isnan(Qf).all(), "a call whose Cholesky gave up a wait must return NaN"
    Q1 = kcholqr_f(Xd)
    torch.cuda.synchronize()
    assert stages.scalars(K, r, cuda)[7].item() == 0.0, "the next call did not clear the wait-error word"
    assert_bits(Q1, Q0, "call after the failure vs before")
    assert_bits(Q1, oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows), "call after the failure vs oracle")


def test_batched_give_up_is_per_call(cuda, zero_spin_limit):
    K, r, n = 768, 512, 3
    Xs = [gen.ttf_uu(K, r, N=K, seed=50 + i).to(cuda) for i in range(n)]
    print("failure path: batched, spin limit 0", flush=True)
    Qs = kcholqr_f_many(Xs)
    torch.cuda.synchronize()
    assert any(torch.isnan(Q).all().item() for Q in Qs), "no matrix of the batch reported its give-up"
    for Q in Qs:
        v = Q.cpu().numpy()
        assert np.isnan(v).all() or np.isfinite(v).all(), "a matrix's Q is partly NaN"
