"""The allocation-free entry point (spanqr_orth_f32_noalloc) through the C ABI: Q bit-identical to spanqr_orth_f32 on
a plan for the same X, on calls in a row whose second is smaller (the fixed workspace keeps the previous call's
contents: flags, dust and tag are rebuilt as needed), under hipGraph capture with calls of another shape between the
replays, and a shape whose workspace exceeds the fixed array is refused with an error."""
import os
import subprocess
import sys

import pytest
import torch

from spanqr_amd import _lib, kcholqr_f
from spanqr_amd.plan import stream_handle
from spanqr_amd.qrbench import gen

from checks import assert_bits

pytestmark = pytest.mark.gpu


def noalloc(X, Q=None):
    K, r = X.shape
    Q = torch.empty_like(X) if Q is None else Q
    _lib.check(_lib.lib().spanqr_orth_f32_noalloc(K, r, X.data_ptr(), r, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                                                  stream_handle(X.device)))
    return Q


def test_noalloc_matches_plan_calls(cuda):
    # the second call smaller than the first; then the first shape again (its dust regenerated) and once more; then
    # a tall shape whose Gram splits are 352 rows (the plain Grams' register-operand kernel)
    for K, r, seed in [(2048, 512, 1), (768, 256, 2), (2048, 512, 3), (2048, 512, 4), (8192, 384, 5)]:
        X = gen.ttf_uu(K, r, N=K, seed=seed).to(cuda)
        print(f"noalloc {K}x{r} seed {seed}", flush=True)
        Qn = noalloc(X)
        Qp = kcholqr_f(X)
        torch.cuda.synchronize()
        assert_bits(Qn, Qp, f"noalloc vs plan call at {K}x{r} (seed {seed})")


def test_noalloc_under_graph_capture(cuda):
    K, r = 768, 512
    X = gen.ttf_uu(K, r, N=K, seed=7).to(cuda)
    Qe = kcholqr_f(X)
    Y = gen.ttf_uu(1024, 256, N=1024, seed=8).to(cuda)
    st = torch.cuda.Stream(cuda)
    st.wait_stream(torch.cuda.current_stream(cuda))
    Qg = torch.empty_like(X)
    with torch.cuda.stream(st):
        noalloc(X, Qg)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("noalloc: graph capture at 768x512", flush=True)
    with torch.cuda.graph(g, stream=st):
        noalloc(X, Qg)
    for rep in range(3):
        Qg.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert_bits(Qg, Qe, f"graph replay {rep}")
        noalloc(Y)                       # another shape between the replays (the replay must rebuild its dust)
        torch.cuda.synchronize()


def test_noalloc_refuses_oversize(cuda):
    X = torch.zeros(32768, 512, device=cuda)
    Q = torch.empty_like(X)
    rc = _lib.lib().spanqr_orth_f32_noalloc(32768, 512, X.data_ptr(), 512, Q.data_ptr(), 512, 5e-7, 1e-7, 1e-8, 2,
                                            stream_handle(cuda))
    assert rc == -1
    assert b"workspace" in _lib.lib().spanqr_last_error()


_FIRST_CALL_CAPTURED = r"""
import sys
import torch
from spanqr_amd import _lib, kcholqr_f
from spanqr_amd.plan import stream_handle
from spanqr_amd.qrbench import gen

K, r = 1024, 256
X = gen.ttf_uu(K, r, N=K, seed=9).to("cuda:0")
Qg = torch.empty_like(X)
st = torch.cuda.Stream()
st.wait_stream(torch.cuda.current_stream())
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=st):   # the process's first allocation-free call: its set-up runs under capture
    _lib.check(_lib.lib().spanqr_orth_f32_noalloc(K, r, X.data_ptr(), r, Qg.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                                                  stream_handle(X.device)))
Qe = kcholqr_f(X)
for rep in range(3):
    Qg.zero_()
    g.replay()
    torch.cuda.synchronize()
    same = torch.equal(Qg.view(torch.int32), Qe.view(torch.int32))
    print(f"replay {rep}: bit-identical {same}", flush=True)
    if not same:
        sys.exit(1)
"""


def test_noalloc_first_call_captured(cuda):
    """the first allocation-free call of a fresh process made under hipGraph capture (the array's device address,
    the kernels' LDS limits and the plan fields are set up while capturing): every replay bit-identical to a plan
    call"""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print("noalloc: first call of a child process under capture", flush=True)
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED], env=env, cwd=root, capture_output=True,
                         text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0, f"child exited with {res.returncode}"
