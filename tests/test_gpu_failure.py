"""The Cholesky's failure path through the C ABI: when one of its bounded waits gives up (forced here from the host by
a spin limit of zero, so every kernel still ends normally), the call's Q comes out NaN and the wait-error word is set;
the next normal call clears the word and is bit-identical to the oracle again. The waits need every workgroup of a
launch resident at once; a give-up is how a violation shows (the reference's cooperative launch fails instead)."""
import numpy as np
import pytest
import torch

import oracle
from spanqr_amd import _lib, borth, kcholqr_f, kcholqr_f_many, set_checked, stages, status
from spanqr_amd.plan import get_plan
from spanqr_amd.qrbench import gen

from checks import assert_bits

pytestmark = pytest.mark.gpu

DEFAULT_LIMIT = 1 << 20


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
    with pytest.raises(_lib.SpanqrError, match="gave up"):
        status(Xd)
    Q1 = kcholqr_f(Xd)
    torch.cuda.synchronize()
    assert stages.scalars(K, r, cuda)[7].item() == 0.0, "the next call did not clear the wait-error word"
    status(Xd)   # the host-side status of the normal call: no error
    assert_bits(Q1, Q0, "call after the failure vs before")
    assert_bits(Q1, oracle.orth(X.numpy(), get_plan(K, r, cuda).split_rows), "call after the failure vs oracle")


def test_checked_mode_raises(cuda):
    """with set_checked(True) a call whose wait gave up raises instead of returning NaN silently; normal calls pass"""
    K, r = 1024, 256
    Xd = gen.ttf_uu(K, r, N=K, seed=4).to(cuda)
    prev = set_checked(True)
    try:
        Q0 = kcholqr_f(Xd)
        print("failure path: checked mode, spin limit 0 at 1024x256", flush=True)
        _lib.lib().spanqr_debug_spin_limit(0)
        try:
            with pytest.raises(_lib.SpanqrError, match="gave up"):
                kcholqr_f(Xd)
        finally:
            _lib.lib().spanqr_debug_spin_limit(DEFAULT_LIMIT)
        Q1 = kcholqr_f(Xd)
    finally:
        set_checked(prev)
    assert_bits(Q1, Q0, "checked call after the failure vs before")


def test_batched_give_up_is_per_call(cuda):
    K, r, n = 768, 512, 3
    Xs = [gen.ttf_uu(K, r, N=K, seed=50 + i).to(cuda) for i in range(n)]
    singles = [kcholqr_f(X) for X in Xs]
    print("failure path: batched, spin limit 0", flush=True)
    _lib.lib().spanqr_debug_spin_limit(0)
    try:
        Qs = kcholqr_f_many(Xs)
        torch.cuda.synchronize()
    finally:
        _lib.lib().spanqr_debug_spin_limit(DEFAULT_LIMIT)
    failed = [bool(torch.isnan(Q).all().item()) for Q in Qs]
    assert any(failed), "no matrix of the batch reported its give-up"
    for Q in Qs:
        v = Q.cpu().numpy()
        assert np.isnan(v).all() or np.isfinite(v).all(), "a matrix's Q is partly NaN"
    with pytest.raises(_lib.SpanqrError, match=f"matrix {failed.index(True)} of the last call"):
        status(Xs)
    # the next batched call at the normal limit clears every matrix's word (the status reads all n) and is
    # bit-identical to the single calls
    Qs = kcholqr_f_many(Xs)
    status(Xs)
    for i, (Q, Qs1) in enumerate(zip(Qs, singles)):
        assert_bits(Q, Qs1, f"batched matrix {i} after the failure vs its single call")


def test_blocked_give_up_is_reported(cuda):
    """the column-blocked path runs kcholf per block, each clearing the wait-error word first: the call's status
    keeps a give-up of any block"""
    K, r = 1024, 768
    Xd = gen.ttf_uu(K, r, N=K, seed=6).to(cuda)
    Q0 = borth(Xd, 256)
    print("failure path: blocked 1024x768, spin limit 0", flush=True)
    _lib.lib().spanqr_debug_spin_limit(0)
    try:
        Qf = borth(Xd, 256)
        torch.cuda.synchronize()
    finally:
        _lib.lib().spanqr_debug_spin_limit(DEFAULT_LIMIT)
    assert torch.isnan(Qf).any()
    with pytest.raises(_lib.SpanqrError, match="gave up"):
        status(Xd)
    Q1 = borth(Xd, 256)
    status(Xd)
    assert_bits(Q1, Q0, "blocked call after the failure vs before")
