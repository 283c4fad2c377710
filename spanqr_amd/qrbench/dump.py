"""Capture real X matrices from a training run as test inputs, in the reference's dump format (qrbench/dump.py).

    from spanqr_amd.qrbench import dump
    uninstall = dump.install("dumps/", calls_per_step=84, steps=(0, 1, 50, 500, 2000))
    ... train ...
    uninstall()

install() wraps the optimizer's orth function (by default `ttf.update._orth_`, the call site the reference patches,
qrbench/dump.py:19-51) in the training process; the training itself is unchanged (the original result is returned).
Each dumped call writes <dir>/s<step>_c<call:03d>_<K>x<r>.pt = {X, V, Q_hh, step, call, layer} (qrbench/dump.py:9-11):
X the input, V the layer's previous basis when the calling frame has one of X's shape, Q_hh the result returned to
training, step/call from the running call count, layer the calling layer's `_ts_idx`. Only the dumped steps
synchronise with the host (the .cpu() copies). The files hold tensors and plain values only, so
gen.real_cases reads them back with torch.load(weights_only=True).
"""
import importlib
import os
import sys

import torch

# the TTF functions whose frames hold the layer (`l`) and its previous basis (`V`) -- qrbench/dump.py:36-38
LAYER_FRAMES = ("ts_layer", "_ts_layer_factored")


def _caller_context(with_v, X):
    """(V, layer) from the nearest calling frame named in LAYER_FRAMES, else (None, None)"""
    f = sys._getframe(2)
    while f is not None and f.f_code.co_name not in LAYER_FRAMES:
        f = f.f_back
    if f is None:
        return None, None
    loc = f.f_locals
    v = loc.get("V")
    V = v.detach().float().cpu() if with_v and torch.is_tensor(v) and tuple(v.shape) == tuple(X.shape) else None
    layer_obj = loc.get("l")
    layer = getattr(layer_obj, "_ts_idx", None) if layer_obj is not None else None
    return V, layer


def install(out_dir, calls_per_step, steps=(0, 1, 50, 500, 2000), max_per_step=None, with_v=True,
            module="ttf.update", attr="_orth_"):
    """Wrap module.attr so that the calls of the given 0-based optimizer steps are dumped. calls_per_step: orth calls
    per optimizer step (110M: 84, 0.8B: 150, 27B: 400 in the reference's runs); max_per_step limits the calls dumped
    per step. module: the module object or its import path. Returns a function that restores the original."""
    if calls_per_step < 1:
        raise ValueError("calls_per_step must be >= 1")
    mod = importlib.import_module(module) if isinstance(module, str) else module
    orig = getattr(mod, attr)
    os.makedirs(out_dir, exist_ok=True)
    wanted = set(steps)
    count = [0]

    def _orth_dump(X):
        Q = orig(X)
        i = count[0]
        count[0] += 1
        step, call = divmod(i, calls_per_step)
        if step in wanted and (max_per_step is None or call < max_per_step):
            V, layer = _caller_context(with_v, X)
            K, r = X.shape
            torch.save(dict(X=X.detach().float().cpu(), V=V, Q_hh=Q.detach().float().cpu(), step=step, call=call,
                            layer=layer), os.path.join(out_dir, f"s{step}_c{call:03d}_{K}x{r}.pt"))
        return Q

    setattr(mod, attr, _orth_dump)

    def uninstall():
        setattr(mod, attr, orig)

    return uninstall
