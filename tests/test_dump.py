"""The real-matrix capture format and loader (qrbench/dump.py, qrbench/gen.py:185-194): the hook writes the
reference's file layout from the TTF call frames, leaves training's result untouched and uninstalls cleanly; the
loader reads both dict and bare-tensor files back (torch.load(weights_only=True)), filtered by shape. CPU only."""
import os
import types

import pytest
import torch

from spanqr_amd.qrbench import dump, gen


class _Layer:
    def __init__(self, idx):
        self._ts_idx = idx


def _fake_ttf():
    mod = types.ModuleType("fake_ttf_update")
    mod._orth_ = lambda X: torch.linalg.qr(X)[0]
    return mod


def ts_layer(mod, l, V, X):     # named as TTF's layer function, whose frame holds `l` and `V`
    return mod._orth_(X)


def test_dump_writes_the_reference_layout(tmp_path):
    mod = _fake_ttf()
    orig = mod._orth_
    g = torch.Generator().manual_seed(1)
    uninstall = dump.install(str(tmp_path), calls_per_step=3, steps=(0, 2), module=mod)
    Xs = [torch.randn(64, 32, generator=g) for _ in range(9)]
    Vs = [torch.linalg.qr(torch.randn(64, 32, generator=g))[0] for _ in range(9)]
    outs = []
    for c, (X, V) in enumerate(zip(Xs, Vs)):
        if c == 4:
            outs.append(mod._orth_(X))                      # no layer frame: V and layer are None
        else:
            outs.append(ts_layer(mod, _Layer(10 + c), V, X))
    uninstall()
    assert mod._orth_ is orig
    for X, Q in zip(Xs, outs):                              # training's result is the original one
        assert torch.equal(Q, torch.linalg.qr(X)[0])
    names = sorted(os.listdir(tmp_path))
    assert names == ["s0_c000_64x32.pt", "s0_c001_64x32.pt", "s0_c002_64x32.pt",
                     "s2_c000_64x32.pt", "s2_c001_64x32.pt", "s2_c002_64x32.pt"]
    d = torch.load(tmp_path / "s2_c001_64x32.pt", weights_only=True)
    assert set(d) == {"X", "V", "Q_hh", "step", "call", "layer"}
    assert d["step"] == 2 and d["call"] == 1 and d["layer"] == 17
    assert torch.equal(d["X"], Xs[7]) and torch.equal(d["V"], Vs[7]) and torch.equal(d["Q_hh"], outs[7])


def test_dump_limits_and_missing_context(tmp_path):
    mod = _fake_ttf()
    uninstall = dump.install(str(tmp_path), calls_per_step=4, steps=(1,), max_per_step=2, with_v=False, module=mod)
    for _ in range(8):
        mod._orth_(torch.randn(40, 16))
    uninstall()
    assert sorted(os.listdir(tmp_path)) == ["s1_c000_40x16.pt", "s1_c001_40x16.pt"]
    d = torch.load(tmp_path / "s1_c000_40x16.pt", weights_only=True)
    assert d["V"] is None and d["layer"] is None
    with pytest.raises(ValueError):
        dump.install(str(tmp_path), calls_per_step=0, module=mod)


def test_real_cases_reads_dumps_back(tmp_path):
    g = torch.Generator().manual_seed(2)
    X1, X2, V1 = torch.randn(96, 64, generator=g), torch.randn(80, 32, generator=g), torch.randn(96, 64, generator=g)
    sub = tmp_path / "run_a"
    sub.mkdir()
    torch.save(dict(X=X1, V=V1, Q_hh=X1, step=0, call=0, layer=3), sub / "s0_c000_96x64.pt")
    torch.save(X2.double(), tmp_path / "bare_80x32.pt")                  # a bare tensor file
    cases = list(gen.real_cases(tmp_path))
    assert [c.name for c in cases] == ["real/bare_80x32", "real/run_a/s0_c000_96x64"]
    assert cases[0].X.dtype == torch.float32 and torch.equal(cases[0].X, X2.float()) and cases[0].ctx == {}
    assert torch.equal(cases[1].X, X1) and torch.equal(cases[1].ctx["V"], V1) and cases[1].hard
    only = list(gen.real_cases(tmp_path, (96, 64)))
    assert [c.name for c in only] == ["real/run_a/s0_c000_96x64"]
    assert list(gen.real_cases(tmp_path / "run_a", (80, 32))) == []


def test_check_cli_parses_shapes():
    from spanqr_amd.qrbench import check
    assert check.parse_shapes("110m") == [(768, 512), (2048, 512)]
    assert check.parse_shapes("1024x256,5120x1024") == [(1024, 256), (5120, 1024)]
    assert check.parse_shapes("bench") == gen.BENCH_SHAPES
