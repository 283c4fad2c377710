"""The real-matrix suite path end to end on the GPU: layers dumped through the capture hook (with this library's orth
as the training-side function) are read back by the loader, the Q each dump recorded is bit-identical to the oracle's
on the dumped X, and the layers pass the check CLI's gates (the reference's hard requirements plus the 2e-7
orthogonality target), including a layer wider than 512 (block Gram-Schmidt)."""
import types

import pytest
import torch

import oracle
from spanqr_amd import orth
from spanqr_amd.plan import get_plan
from spanqr_amd.qrbench import check, dump, gen

from checks import assert_bits

pytestmark = pytest.mark.gpu


def ts_layer(mod, l, V, X):     # named as TTF's layer function
    return mod._orth_(X)


def test_dumped_layers_pass_the_check(cuda, tmp_path):
    mod = types.ModuleType("fake_ttf_update")
    mod._orth_ = orth
    shapes = [(1024, 256), (768, 512), (1024, 768)]
    uninstall = dump.install(str(tmp_path), calls_per_step=len(shapes), steps=(0,), module=mod)
    for n, (K, r) in enumerate(shapes):
        X = gen.bench_input(K, r, seed=20 + n).to(cuda)
        V = torch.linalg.qr(torch.randn(K, r, device=cuda))[0]
        print(f"dump {K}x{r}", flush=True)
        Q = ts_layer(mod, types.SimpleNamespace(_ts_idx=n), V, X)
        assert Q.shape == X.shape
    uninstall()
    cases = list(gen.real_cases(tmp_path))
    assert len(cases) == 3
    for p in sorted(tmp_path.rglob("*.pt")):
        d = torch.load(p, map_location="cpu", weights_only=True)
        X = d["X"].numpy()
        K, r = X.shape
        want = oracle.borth(X) if r > 512 else oracle.orth(X, get_plan(K, r, cuda).split_rows)
        assert_bits(d["Q_hh"], want, f"dumped layer {p.name} vs oracle")
    rc = check.main(["--real", str(tmp_path), "--real-only", "--target",
                     "--shapes", ",".join(f"{K}x{r}" for K, r in shapes)])
    assert rc == 0
