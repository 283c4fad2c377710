"""Checks that pin the CPU oracle (oracle/) to the reference's algorithm without running the reference.

Each check returns a list of failure messages (empty: pinned). They compare the oracle with what fixes the answer
independently of the oracle's own code: torch's CPU evaluation of the reference's own expressions
(candidates/kcholqr.py:29-30, :16-23, :107-109), fp64 textbook linear algebra (Cholesky, triangular solve, Gram)
under rounding-error bounds, closed forms and special cases (zero Gram, clamped pivots, NaN pivots), invariants
(exact power-of-2 scaling, symmetry, unit dust columns) and the published splitmix64 sequence. tests/test_oracle.py
runs them on the oracle (all must pass) and on copies of the oracle built with a planted defect (each defect must
make at least one check fail).
"""
import math

import numpy as np
import torch

import oracle

U32 = 2.0 ** -24
F32 = np.float32


def _ulps(got, ref):
    ref = np.asarray(ref, np.float64)
    return np.abs(np.asarray(got, np.float64) - ref) / np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)


# ---- power-of-2 scale (kcholqr.py:29-30) ----

def torch_pow2_scale(m):
    """the reference's expression, evaluated by torch on the CPU (fp32)"""
    t = torch.as_tensor(np.asarray(m, np.float32))
    return torch.where(t > 0, torch.exp2(-torch.round(torch.log2(t.clamp_min(1e-38)))), torch.ones_like(t)).numpy()


def scale_windows():
    """every float whose log2 lies near a half-integer (mantissa near sqrt(2)) for all 254 exponents, plus the
    binade ends: where round(log2) is decided"""
    mant = np.concatenate([np.arange(0x3504C0, 0x350530, dtype=np.uint32),
                           np.array([0, 1, 0x200000, 0x400000, 0x7FFFFF], np.uint32)])
    e = np.arange(1, 255, dtype=np.uint32)
    return ((e[:, None] << np.uint32(23)) | mant[None, :]).ravel().view(np.float32)


def check_scale():
    f = []
    x = scale_windows()
    got = np.array([oracle.pow2_scale(v) for v in x], np.float32)
    want = torch_pow2_scale(x)
    bad = np.nonzero(got != want)[0]
    if len(bad):
        f.append(f"pow2_scale differs from torch's round(log2) at {len(bad)} of {len(x)} values, e.g. "
                 f"m={x[bad[0]]!r}: {got[bad[0]]} vs {want[bad[0]]}")
    known = {0.0: 1.0, float("nan"): 1.0, float("inf"): 0.0, 1.0: 1.0, 2.0 ** 20: 2.0 ** -20, 1.25 * 2.0 ** 7: 2.0 ** -7,
             1.5 * 2.0 ** 7: 2.0 ** -8, 1.5 * 2.0 ** -9: 2.0 ** 8, 1e-40: 2.0 ** 126, 1e-25: 2.0 ** 83, 1e25: 2.0 ** -83}
    for m, s in known.items():
        if oracle.pow2_scale(m) != F32(s):
            f.append(f"pow2_scale({m}) = {oracle.pow2_scale(m)}, expected {s}")
    # invariant: s is a power of 2 and max|s x| lands in [2^-1/2, 2^1/2] (up to the half-way band)
    rng = np.random.default_rng(1)
    m = (10.0 ** rng.uniform(-37, 37, 2000)).astype(np.float32)
    for v in m:
        s = float(oracle.pow2_scale(v))
        if math.frexp(s)[0] != 0.5 or not (2 ** -0.5 * (1 - 1e-6) <= v * s <= 2 ** 0.5 * (1 + 1e-6)):
            f.append(f"pow2_scale({v}) = {s} breaks the invariant")
            break
    return f


def check_scale_rounding_margin():
    """the oracle and the kernels take fp32(log2) from a double log2; near the half-integers (where it decides the
    result) the double value must sit far from every fp32 rounding boundary, so any log2 within a few double ulps
    gives the same fp32 value"""
    x = scale_windows()
    l = np.log2(x.astype(np.float64))
    y = l.astype(np.float32)
    lo = np.nextafter(y, np.float32(-np.inf)).astype(np.float64)
    hi = np.nextafter(y, np.float32(np.inf)).astype(np.float64)
    yd = y.astype(np.float64)
    gap = np.minimum(np.abs(l - (yd + lo) / 2), np.abs(l - (yd + hi) / 2))
    worst = float((gap / np.spacing(np.abs(l))).min())
    return [] if worst > 64 else [f"double log2 within {worst} double ulps of an fp32 rounding boundary"]


def check_amax():
    """max|x| (torch.linalg.vector_norm(X, ord=inf) at candidates/kcholqr.py:102) against torch's own CPU evaluation
    of that expression: the largest magnitude carried by a negative entry, +-inf, NaN (propagates), all -0.0,
    subnormal-only, and a row stride wider than r (columns past r are not part of X)"""
    f = []
    rng = np.random.default_rng(11)
    cases = {}
    X = rng.standard_normal((37, 24)).astype(np.float32)
    cases["random"] = X
    Y = X.copy()
    Y[5, 7] = -50.0
    cases["negative maximum"] = Y
    Y = X.copy()
    Y[0, 0] = -np.inf
    cases["-inf"] = Y
    Y = X.copy()
    Y[36, 23] = np.inf
    cases["+inf"] = Y
    Y = X.copy()
    Y[3, 2] = np.nan
    Y[4, 4] = np.inf
    cases["nan"] = Y
    cases["all -0"] = np.full((8, 16), -0.0, np.float32)
    cases["subnormal"] = (rng.standard_normal((16, 8)) * 1e-40).astype(np.float32)
    for name, A in cases.items():
        want = float(torch.linalg.vector_norm(torch.from_numpy(A), ord=float("inf")))
        got = float(oracle.amax(A))
        same = (math.isnan(want) and math.isnan(got)) or (want == got and math.copysign(1, want) == math.copysign(1, got))
        if not same:
            f.append(f"amax({name}) = {got!r}, torch.linalg.vector_norm(inf) = {want!r}")
    W = np.zeros((20, 12), np.float32)
    W[:, :8] = rng.standard_normal((20, 8))
    W[:, 8:] = -1e9                                   # outside the 8 columns of X
    got = float(oracle.lib().spqo_amax(W, 12, 20, 8))
    want = float(torch.linalg.vector_norm(torch.from_numpy(W[:, :8].copy()), ord=float("inf")))
    if got != want:
        f.append(f"amax with a row stride wider than r reads past the columns: {got} vs {want}")
    return f


# ---- pivot reciprocal square root (chol.cu:45 uses rsqrtf) ----

def check_rsqrt():
    rng = np.random.default_rng(2)
    x = (10.0 ** rng.uniform(-37.9, 38, 5000)).astype(np.float32)
    x = np.concatenate([x, np.float32([1e-30, 1.0, 2.0, 4.0, 0.25, 3.0, 1e-8])])
    got = np.array([oracle.rsqrt(v) for v in x], np.float32)
    err = _ulps(got, 1.0 / np.sqrt(x.astype(np.float64)))
    return [] if err.max() <= 2.5 else [f"rsqrt error {err.max():.2f} ulp > 2.5"]


# ---- dust (this project's generator, seeded with the reference's 20261018, kcholqr.py:83-89) ----

MASK64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def mix64(z):
    """splitmix64's output function (Steele, Lea, Flood 2014; Vigna's splitmix64.c)"""
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def dust_spec(K, r, seed=20261018):
    """the generator's written definition, in exact integer and double arithmetic"""
    key = mix64(seed)
    raw = np.empty((K, r), np.float32)
    for k in range(K):
        for c in range(r):
            n = k * r + c
            S = 0
            for j in range(6):
                w = mix64((key + (6 * n + j + 1) * GOLDEN) & MASK64)
                S += (w & 0xFFFFFFFF) + (w >> 32)
            raw[k, c] = np.float32(math.ldexp(float(S - 6 * 0xFFFFFFFF), -32))
    return raw, None


def check_dust():
    f = []
    # splitmix64 seeded with 0: first outputs as published
    state, outs = 0, []
    for _ in range(2):
        state = (state + GOLDEN) & MASK64
        outs.append(mix64(state))
    if outs != [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]:
        f.append("splitmix64 restatement does not reproduce the published sequence")
    K, r = 7, 5
    raw, _ = dust_spec(K, r)
    nrm = []
    for c in range(r):
        acc = 0.0
        for k in range(K):                      # ascending k, in double
            acc += float(raw[k, c]) * float(raw[k, c])
        nrm.append(math.sqrt(acc))
    nrm = np.array(nrm)
    Z = oracle.dust(K, r)
    want = (raw.astype(np.float64) / nrm).astype(np.float32)
    if not np.array_equal(Z, want):
        f.append(f"dust differs from its definition (max diff {np.abs(Z - want).max():.3e})")
    Zb = oracle.dust(512, 64)
    cn = np.sqrt((Zb.astype(np.float64) ** 2).sum(axis=0))
    if not np.abs(cn - 1).max() <= 1e-6:
        f.append(f"dust columns are not unit (max |norm - 1| {np.abs(cn - 1).max():.2e})")
    zk = Zb.astype(np.float64) * math.sqrt(512)
    if not (abs(zk.mean()) <= 0.02 and abs(zk.var() - 1) <= 0.03):
        f.append(f"dust entries not ~N(0, 1/K): mean {zk.mean():.3f} var {zk.var():.3f}")
    return f


# ---- Gram (tri.py:255-297, 324-375) ----

def check_gram():
    f = []
    rng = np.random.default_rng(3)
    # ragged last split (200 = 3 x 64 + 8); r = 96 and 32: the last 64-column tile is half outside X (its columns
    # read as 0, entries past r neither stored nor counted in the norm partials). The norm partials come in both
    # groupings: one per upper 32x32 tile for short X with many tiles (K <= 1024, r >= 448: the last two), 16 per
    # upper 64x64 tile otherwise
    for K, r, KS in ((200, 128, 64), (200, 96, 64), (150, 32, 64), (600, 480, 320), (460, 448, 256)):
        X = rng.standard_normal((K, r)).astype(np.float32)
        X[:, 5] *= 1e3
        G64 = X.astype(np.float64).T @ X.astype(np.float64)
        A64 = np.abs(X.astype(np.float64)).T @ np.abs(X.astype(np.float64))
        for kahan, c in ((True, 4.0), (False, KS + 8.0)):
            G, npart = oracle.gram(X, KS, kahan)
            ratio = (np.abs(G - G64) / (A64 * U32)).max()
            if not ratio <= c:
                f.append(f"gram(r={r}, kahan={kahan}) error {ratio:.1f} u|X|^T|X| > {c}")
            if not np.array_equal(G, G.T):
                f.append(f"gram (r={r}) not exactly symmetric")
            fro2 = float((G.astype(np.float64) ** 2).sum())
            nt, nb = -(-r // 64), r // 32
            want = nb * (nb + 1) // 2 if oracle.gram_short(K, r) else 16 * nt * (nt + 1) // 2
            if npart.size != want or oracle.gram_short(K, r) != (K <= 1024 and r >= 448):
                f.append(f"gram({K}x{r}): {npart.size} norm partials, expected {want}")
            if not abs(npart.sum() - fro2) <= 1e-12 * fro2:
                f.append(f"norm partials (r={r}) do not sum to ||G||_F^2")
            if not abs(float(oracle.norm(npart)) - math.sqrt(fro2)) <= 2 * U32 * math.sqrt(fro2):
                f.append(f"norm() (r={r}) is not ||G||_F")
    K, r, KS = 200, 128, 64
    X = rng.standard_normal((K, r)).astype(np.float32)
    X[:, 5] *= 1e3
    # one long split (128 chunks of 32 rows): Kahan compensation across chunks keeps the error near 1 u|X|^T|X|
    # where a plain chain reaches tens of u
    X2 = (rng.standard_normal((4096, 64)) + 3.0).astype(np.float32)
    X2d = X2.astype(np.float64)
    G2, _ = oracle.gram(X2, 4096, True)
    ratio = (np.abs(G2 - X2d.T @ X2d) / (np.abs(X2d).T @ np.abs(X2d) * U32)).max()
    if not ratio <= 4.0:
        f.append(f"Kahan Gram over one 4096-row split: error {ratio:.1f} u|X|^T|X| > 4")
    # scaling by a power of 2 on load is exact
    s = F32(2.0 ** -7)
    Gs, _ = oracle.gram(X, KS, True, s=s)
    Gp, _ = oracle.gram(X * s, KS, True)
    if not np.array_equal(Gs, Gp):
        f.append("gram with scale on load differs from the Gram of the scaled matrix")
    if oracle.gram_splits(200, 64) != 4 or oracle.gram_splits(256, 64) != 4:
        f.append("gram_splits is not ceil(K / KS)")
    return f


# ---- shift and clamp floor (kcholqr.py:107-109) ----

def check_shift():
    f = []
    rng = np.random.default_rng(4)
    G = rng.standard_normal((64, 64)).astype(np.float32)
    nrm = F32(123.456)
    Gs, tau = oracle.shift(G, nrm)
    t = torch.from_numpy(G.copy())
    t.diagonal().add_(torch.tensor(1e-7, dtype=torch.float32) * torch.tensor(float(nrm), dtype=torch.float32))
    tt = torch.tensor(1e-8, dtype=torch.float32) * torch.tensor(float(nrm), dtype=torch.float32) + 1e-30
    if not np.array_equal(Gs, t.numpy()):
        f.append("shift differs from G.diagonal().add_(alpha * nrm)")
    if tau != F32(tt.item()):
        f.append(f"tau {tau} differs from tau * nrm + 1e-30 = {tt.item()}")
    return f


# ---- clamped Cholesky (chol.cu:115-271) ----

def _spd(r, cond, seed):
    rng = np.random.default_rng(seed)
    Qm, _ = np.linalg.qr(rng.standard_normal((r, r)))
    s = np.logspace(0, -math.log10(cond), r)
    return ((Qm * s) @ Qm.T).astype(np.float32)


def check_chol():
    f = []
    r = 128
    G = _spd(r, 100.0, 5)
    L, Li = oracle.chol(G, 1e-30)
    L64 = torch.linalg.cholesky(torch.from_numpy(G.astype(np.float64))).numpy()
    rel = np.abs(L - L64).max() / np.abs(L64).max()
    if not rel <= 1e-5:
        f.append(f"chol differs from fp64 Cholesky by {rel:.2e}")
    if not np.abs(np.triu(L, 1)).max() == 0:
        f.append("chol: upper triangle not zero")
    res = np.abs(L.astype(np.float64) @ L.T - G).max() / np.abs(G).max()
    if not res <= 1e-5:
        f.append(f"chol residual {res:.2e}")
    for j in range(r // 32):
        Ljj = L[32 * j:32 * j + 32, 32 * j:32 * j + 32].astype(np.float64)
        e = np.abs(Li[32 * j:32 * j + 32].astype(np.float64) @ Ljj - np.eye(32)).max()
        if not e <= 1e-4:
            f.append(f"Li block {j} is not the inverse of the diagonal tile ({e:.2e})")
            break
        if not np.abs(np.triu(Li[32 * j:32 * j + 32], 1)).max() == 0:
            f.append("Li not lower triangular")
            break
    # zero Gram: every pivot clamps to tau -> L = sqrt(tau) I
    Lz, Liz = oracle.chol(np.zeros((64, 64), np.float32), 1e-30)
    if not (np.abs(np.diag(Lz) / 1e-15 - 1).max() <= 1e-6 and np.abs(Lz - np.diag(np.diag(Lz))).max() == 0):
        f.append("chol of zero is not sqrt(tau) I")
    if not np.abs(np.diag(Liz[:32]) * 1e-15 - 1).max() <= 1e-6:
        f.append("Li of zero Gram is not I / sqrt(tau)")
    # rank 32 of 96: pivots 33.. clamp to tau (chosen far above the rounding noise)
    rng = np.random.default_rng(6)
    B = rng.standard_normal((96, 32)).astype(np.float64)
    Gr = (B @ B.T).astype(np.float32)
    tau = 1e-3 * float(np.abs(Gr).max())
    Lr, _ = oracle.chol(Gr, tau)
    d = np.diag(Lr)[32:]
    if not np.abs(d / math.sqrt(tau) - 1).max() <= 1e-5:
        f.append("clamped pivots of a rank-deficient Gram are not sqrt(tau)")
    # NaN pivot -> tau (fmaxf ignores NaN, chol.cu:9)
    Gn = _spd(64, 10.0, 7)
    Gn[3, 3] = np.nan
    Ln, _ = oracle.chol(Gn, 0.5)
    if not abs(Ln[3, 3] / math.sqrt(0.5) - 1) < 1e-6:
        f.append("NaN pivot not clamped to tau")
    return f


# ---- triangular solve (tri.py:378-412) ----

def check_trsm():
    f = []
    r, K = 128, 100
    G = _spd(r, 50.0, 8)
    L, Li = oracle.chol(G, 1e-30)
    rng = np.random.default_rng(9)
    A = rng.standard_normal((K, r)).astype(np.float32)
    Y = oracle.trsm(A, L, Li)
    Y64 = torch.linalg.solve_triangular(torch.from_numpy(L.astype(np.float64)),
                                        torch.from_numpy(A.astype(np.float64)).T, upper=False).T.numpy()
    rel = np.abs(Y - Y64).max() / np.abs(Y64).max()
    if not rel <= 1e-5:
        f.append(f"trsm differs from fp64 solve_triangular by {rel:.2e}")
    # pass-1 operand fmaf(eps, z, s x): with eps = 0 it is exactly s x
    s = F32(0.25)
    Z = oracle.dust(K, r)
    Y1 = oracle.trsm(A, L, Li, s=s, Z=Z, eps=0.0)
    Y0 = oracle.trsm(A * s, L, Li)
    if not np.array_equal(Y1, Y0):
        f.append("trsm pass-1 operand with eps = 0 is not s * x")
    Ye = oracle.trsm(A, L, Li, s=s, Z=Z, eps=1e-3)
    Ye64 = torch.linalg.solve_triangular(torch.from_numpy(L.astype(np.float64)),
                                         torch.from_numpy((0.25 * A + 1e-3 * Z).astype(np.float64)).T,
                                         upper=False).T.numpy()
    if not np.abs(Ye - Ye64).max() / np.abs(Ye64).max() <= 1e-5:
        f.append("trsm pass-1 operand is not s x + eps z")
    return f


# ---- Newton-Schulz polish (kcholqr.py:16-23) ----

def check_ns():
    f = []
    rng = np.random.default_rng(10)
    K, r = 300, 64
    Q0, _ = np.linalg.qr(rng.standard_normal((K, r)))
    E = 1e-3 * rng.standard_normal((r, r))
    Y = (Q0 @ (np.eye(r) + (E + E.T) / 2)).astype(np.float32)
    G = (Y.astype(np.float64).T @ Y).astype(np.float32)
    D = oracle.ns_D(G)
    Dt = torch.eye(r).sub_(torch.from_numpy(G)).mul_(0.5).numpy()     # the reference's expression
    if not np.array_equal(D, Dt):
        f.append("ns_D differs from eye(r).sub_(G).mul_(0.5)")
    Q = oracle.ns_apply(Y, D)
    Q64 = Y.astype(np.float64) + Y.astype(np.float64) @ D.astype(np.float64)
    if not np.abs(Q - Q64).max() <= 4 * U32 * np.abs(Q64).max():
        f.append("ns_apply is not Y + Y D")
    e0 = np.abs(Y.astype(np.float64).T @ Y - np.eye(r)).max()
    e1 = np.abs(Q.astype(np.float64).T @ Q - np.eye(r)).max()
    if not e1 < max(10 * e0 ** 2, 2e-6):
        f.append(f"one polish step does not square the orthogonality error ({e0:.2e} -> {e1:.2e})")
    return f


# ---- whole call on small shapes ----

def check_orth_small():
    from spanqr_amd.qrbench import gen, metrics
    f = []
    K, r = 256, 128
    for name in ("mixed_c2", "mixed_c8", "zero", "rank_half", "huge_1e25"):
        c = next(gen.make_cases(K, r, [name], (0,)))
        Q = oracle.orth(c.X.numpy(), 64)
        ref = metrics.reference(c.X)
        res = metrics.assess(torch.from_numpy(Q), c.X, ref)
        hh = metrics.assess(metrics.householder(c.X), c.X, ref)
        fails = res.failures(span_ref=hh.span_n, orth_tol=metrics.ORTH_TOL_TARGET)
        if fails:
            f.append(f"orth {name}: {fails}")
        if name == "mixed_c2":
            # thin-QR uniqueness: on a well-conditioned X the result is Householder's Q up to column signs
            Qh, Rh = torch.linalg.qr(c.X.double())
            Qh = (Qh * torch.sign(torch.diagonal(Rh))).numpy()
            if not np.abs(Q - Qh).max() <= 1e-4:
                f.append(f"orth mixed_c2 is not the thin-QR Q ({np.abs(Q - Qh).max():.2e})")
    return f


# ---- column-blocked path (kbig.py:69-95) ----

def check_split_rule():
    """the split rule's own invariants: KS a multiple of 32, no empty split, at most ceil(512 / U) splits and at most
    ceil(K / 128)"""
    f = []
    for K in (1, 31, 32, 127, 128, 129, 1000, 4096, 17408, 100000):
        for U in (1, 4, 8, 10, 36, 136, 240):
            KS = oracle.split_rows(K, U)
            S = oracle.gram_splits(K, KS)
            if KS % 32 or KS <= 0:
                f.append(f"split_rows({K}, {U}) = {KS} not a positive multiple of 32")
            elif S > max(1, -(-512 // U)) or S > max(1, -(-K // 128)) or (S - 1) * KS >= K:
                f.append(f"split_rows({K}, {U}) = {KS}: {S} splits")
    return f


def check_xgram():
    """P^T C against fp64 under the fp32 chain bound, exactly on integer data, and split-count independent on it"""
    f = []
    rng = np.random.default_rng(11)
    for K, j, KS in ((300, 256, 128), (1000, 512, 256), (77, 256, 96)):
        P = rng.standard_normal((K, j)).astype(np.float32)
        C = rng.standard_normal((K, 256)).astype(np.float32)
        T = oracle.xgram(P, C, KS).astype(np.float64)
        T64 = P.astype(np.float64).T @ C
        bound = (KS + 2) * U32 * (np.abs(P).astype(np.float64).T @ np.abs(C))
        if not (np.abs(T - T64) <= bound).all():
            f.append(f"xgram K={K} j={j}: not P^T C")
        Pi = rng.integers(-8, 9, (K, j)).astype(np.float32)
        Ci = rng.integers(-8, 9, (K, 256)).astype(np.float32)
        Ti = Pi.astype(np.int64).T @ Ci.astype(np.int64)
        for ks in (KS, 32):
            if not np.array_equal(oracle.xgram(Pi, Ci, ks), Ti.astype(np.float32)):
                f.append(f"xgram K={K} j={j} KS={ks}: integer product not exact")
    return f


def check_project():
    """C - P P^T C: fp64 agreement, P^T Out ~ 0 for orthonormal P, a vector in span(P) removed, one orthogonal to
    it kept"""
    f = []
    rng = np.random.default_rng(12)
    K, j = 600, 512
    P = np.linalg.qr(rng.standard_normal((K, j)))[0].astype(np.float32)
    C = rng.standard_normal((K, 256)).astype(np.float32)
    KS = oracle.split_rows(K, (j // 64) * 4)
    Out = oracle.project(P, C, KS).astype(np.float64)
    P64 = P.astype(np.float64)
    ref = C - P64 @ (P64.T @ C)
    if not np.abs(Out - ref).max() <= 1e-4:
        f.append(f"project: not C - P P^T C ({np.abs(Out - ref).max():.2e})")
    if not np.abs(P64.T @ Out).max() <= 1e-4:
        f.append("project: result not orthogonal to P")
    inside = (P64 @ rng.standard_normal((j, 256))).astype(np.float32)
    if not np.abs(oracle.project(P, inside, KS)).max() <= 1e-4 * np.abs(inside).max():
        f.append("project: a matrix in span(P) is not removed")
    perp = (C.astype(np.float64) - P64 @ (P64.T @ C)).astype(np.float32)
    if not np.abs(oracle.project(P, perp, KS) - perp).max() <= 1e-4 * np.abs(perp).max():
        f.append("project: a matrix orthogonal to P is changed")
    return f


def _thin_q(X):
    Qh, Rh = np.linalg.qr(X.astype(np.float64))
    return Qh * np.sign(np.diag(Rh))


def check_borth():
    """borth on small shapes: on a well-conditioned X it is the thin-QR Q (BCGS with positive-diagonal block
    factors gives X = Q R, R upper triangular with a positive diagonal, which fixes Q); X = 0 gives block j the span of
    the dust's columns j.. with the earlier blocks removed; a repeated block is completed, never zero or NaN"""
    f = []
    rng = np.random.default_rng(13)
    K, r = 1000, 768
    X = rng.standard_normal((K, r)).astype(np.float32)
    Q = oracle.borth(X).astype(np.float64)
    if not np.abs(Q - _thin_q(X)).max() <= 1e-4:
        f.append(f"borth: not the thin-QR Q on a well-conditioned X ({np.abs(Q - _thin_q(X)).max():.2e})")
    for name, Xc in (("zero", np.zeros((K, r), np.float32)),
                     ("repeated block", np.concatenate([X[:, :512], X[:, :256]], axis=1))):
        Q = oracle.borth(Xc).astype(np.float64)
        if not np.isfinite(Q).all() or not np.abs(Q.T @ Q - np.eye(r)).max() <= 1e-6:
            f.append(f"borth {name}: Q not orthonormal")
            continue
        if name == "zero":
            Z = oracle.dust(K, r).astype(np.float64)
            for j in range(0, r, 256):
                Zp = Z[:, j:j + 256] - Q[:, :j] @ (Q[:, :j].T @ Z[:, j:j + 256])
                Qj = Q[:, j:j + 256]
                if not np.abs(Zp - Qj @ (Qj.T @ Zp)).max() <= 1e-5 * np.abs(Zp).max():
                    f.append(f"borth zero: block {j // 256} does not span its projected dust slice")
        else:
            Qh = _thin_q(Xc[:, :512])
            if not np.abs(Q[:, :512] - Qh).max() <= 1e-4:
                f.append("borth repeated block: leading blocks are not the thin-QR Q")
    return f


def check_borth_composition():
    """kbig.py:85-93 step by step from the pieces pinned above, for orth's b = 256 and for b = 128 with and without
    the reorthogonalisation: s from all of X, each block twice projected, _kf with its dust slice, and with reorth
    once more projected and _kf again"""
    f = []
    rng = np.random.default_rng(14)
    K, r = 800, 768
    X = (rng.standard_normal((K, r)) * np.exp(rng.uniform(-3, 3, r))).astype(np.float32)
    s = oracle.pow2_scale(oracle.amax(X))
    Z = oracle.dust(K, r)
    for b, reorth in ((256, True), (128, True), (128, False)):
        Q = oracle.borth(X, b, reorth)
        KSb = oracle.gram_rows(K, b)
        R = np.empty_like(X)
        for j in range(0, r, b):
            W = X[:, j:j + b] * s
            if j:
                KSp = oracle.split_rows(K, (j // 64) * (b // 64))
                W = oracle.project(R[:, :j], oracle.project(R[:, :j], W, KSp), KSp)
            W = oracle.orth_dust(W, Z[:, j:j + b], KSb)
            if j and reorth:
                W = oracle.orth_dust(oracle.project(R[:, :j], W, KSp), Z[:, j:j + b], KSb)
            R[:, j:j + b] = W
        if not np.array_equal(Q.view(np.uint32), R.view(np.uint32)):
            f.append(f"borth(b={b}, reorth={reorth}) is not kbig.py's composition of scale, projections and _kf")
    # b = 128 without the reorthogonalisation still gives the thin-QR Q on a well-conditioned X
    Xw = rng.standard_normal((1000, 512)).astype(np.float32)
    Qw = oracle.borth(Xw, 128, False).astype(np.float64)
    if not np.abs(Qw - _thin_q(Xw)).max() <= 1e-4:
        f.append("borth(b=128, reorth=False): not the thin-QR Q on a well-conditioned X")
    return f


# ---- fp64 Cholesky (kchol.py:47-57, chol.cu:278-281) ----

def check_rsqrt64():
    """the fp64 pivot reciprocal square root within 3 ulp of 1/sqrt in extended precision over 1e-300..1e300"""
    x = np.logspace(-300, 300, 4001)
    y = np.array([oracle.rsqrt64(v) for v in x])
    ref = (1 / np.sqrt(x.astype(np.longdouble))).astype(np.float64)
    ulp = np.abs(y - ref) / np.spacing(ref)
    return [] if ulp.max() <= 3 else [f"rsqrt64 off by {ulp.max():.1f} ulp"]


def check_chol64():
    """fp64 LAPACK Cholesky (clamp inactive), residual, Li L_jj = I, zero G -> sqrt(tau) I, NaN pivot -> tau,
    rank deficiency clamped, fp32 copies the rounded fp64 values"""
    f = []
    rng = np.random.default_rng(15)
    for r in (64, 256):
        X = rng.standard_normal((r + 40, r))
        G = X.T @ X
        L, Li, Lf, Lif = oracle.chol64(G, 1e-12)
        L0 = np.linalg.cholesky(G)
        if not np.abs(L - L0).max() <= 1e-12 * np.abs(L0).max():
            f.append(f"chol64 r={r}: not LAPACK's factor ({np.abs(L - L0).max():.2e})")
        if not np.abs(L @ L.T - G).max() <= 1e-13 * np.abs(G).max():
            f.append(f"chol64 r={r}: residual")
        for j in range(r // 32):
            Ljj = L[32 * j:32 * j + 32, 32 * j:32 * j + 32]
            if not np.abs(Li[32 * j:32 * j + 32] @ Ljj - np.eye(32)).max() <= 1e-12 * max(1.0, np.abs(Li).max()):
                f.append(f"chol64 r={r}: Li is not the diagonal tile's inverse")
                break
        if not (np.array_equal(Lf, L.astype(np.float32)) and np.array_equal(Lif, Li.astype(np.float32))):
            f.append("chol64: fp32 copies are not the rounded fp64 values")
        if not np.all(np.triu(L, 1) == 0):
            f.append("chol64: upper triangle not zero")
    tau = 1e-20
    L, Li, _, _ = oracle.chol64(np.zeros((64, 64)), tau)
    if not np.allclose(L, np.sqrt(tau) * np.eye(64), rtol=1e-15, atol=0):
        f.append("chol64: zero G does not give sqrt(tau) I")
    G = rng.standard_normal((96, 64))
    G = G.T @ G
    G[5, 5] = np.nan
    L, _, _, _ = oracle.chol64(G, 1e-3)
    if not abs(L[5, 5] - np.sqrt(1e-3)) <= 1e-15 or not np.isfinite(L[:5, :5]).all():
        f.append("chol64: a NaN pivot is not clamped to tau")
    B = rng.standard_normal((64, 16))
    L, _, _, _ = oracle.chol64(B @ B.T, 1e-10)
    if not (np.diag(L)[16:] <= 2 * np.sqrt(1e-10)).all():
        f.append("chol64: rank-deficient pivots are not clamped")
    return f


ALL = [check_amax, check_scale, check_scale_rounding_margin, check_rsqrt, check_dust, check_gram, check_shift, check_chol,
       check_trsm, check_ns, check_orth_small, check_split_rule, check_xgram, check_project, check_borth,
       check_borth_composition, check_rsqrt64, check_chol64]
