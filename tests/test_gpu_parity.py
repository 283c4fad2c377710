"""MI355X kernels against the CPU oracle, bit for bit, stage by stage and end to end.

Every output element of the HIP kernels follows the operation order of oracle/kcholf_oracle.c (an fp32 MFMA chain
on gfx950 rounds like a sequential fmaf chain), so equality is exact: compared as uint32 bit patterns.
"""
import numpy as np
import pytest
import torch

import oracle
from spanqr_amd import orth, stages
from spanqr_amd.plan import get_plan
from spanqr_amd.qrbench import gen

pytestmark = pytest.mark.gpu


def bits(t):
    a = t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint64)


def assert_bits(gpu, ref, what):
    g, o = bits(gpu), bits(ref)
    if not np.array_equal(g, o):
        gf = (gpu.detach().cpu().numpy() if isinstance(gpu, torch.Tensor) else gpu).astype(np.float64)
        of = np.asarray(ref, np.float64)
        bad = np.argwhere(g != o)
        raise AssertionError(f"{what}: {len(bad)} of {g.size} elements differ; first at {bad[0].tolist()}: "
                             f"gpu {gf[tuple(bad[0])]!r} oracle {of[tuple(bad[0])]!r}; max abs diff "
                             f"{np.abs(gf - of).max():.3e}")


def case_x(K, r, name="mixed_c4", seed=0):
    return next(gen.make_cases(K, r, [name], (seed,))).X


SHAPES = [(256, 64), (256, 128), (384, 256), (768, 512)]
# r a multiple of 32 but not of 64 (kcholqr.py:98-99 runs kcholf there too): the last 64-column Gram / NS tile is
# half outside X, and an odd number of 32-column blocks in the Cholesky and the solve
SHAPES32 = [(100, 32), (300, 96), (512, 160), (640, 224), (1000, 480)]
# kcholf at full width above 512 columns (orth.py:20 for r not a multiple of 256; kcholqr_f at any multiple of 32):
# tile rows of up to 32 tiles over up to six owner workgroups each, four column blocks per solve wavefront
SHAPESW = [(600, 544), (1100, 640), (2000, 800), (1024, 992), (1100, 1024)]
# splits of 352 rows (the plain Gram's register-operand kernel), one with a ragged last chunk and r % 64 == 32
SHAPESL = [(8192, 384), (8100, 352), (16700, 224)]


@pytest.mark.parametrize("K,r", SHAPES)
def test_dust_on_device(cuda, K, r):
    print(f"dust {K}x{r}", flush=True)
    Z = stages.dust(K, r, cuda)
    assert_bits(Z, oracle.dust(K, r), "dust")


@pytest.mark.parametrize("K,r", SHAPES + SHAPES32 + SHAPESW + SHAPESL)
@pytest.mark.parametrize("kahan", [True, False])
def test_gram(cuda, K, r, kahan):
    print(f"gram {K}x{r} kahan={kahan}", flush=True)
    X = case_x(K, r)
    plan = get_plan(K, r, cuda)
    G, npart = stages.gram(X.to(cuda), kahan)
    Go, npo = oracle.gram(X.numpy(), plan.split_rows, kahan)
    assert_bits(G, Go, "G")
    assert_bits(npart, npo, "norm partials")


@pytest.mark.parametrize("K,r", SHAPES + SHAPES32 + SHAPESW)
def test_gram_scaled(cuda, K, r):
    print(f"gram scaled {K}x{r}", flush=True)
    X = case_x(K, r, "huge_1e25")
    plan = get_plan(K, r, cuda)
    Xd = X.to(cuda)
    stages.amax(Xd)
    G, npart = stages.gram(Xd, True, use_scale=True)
    s = oracle.pow2_scale(oracle.amax(X.numpy()))
    Go, npo = oracle.gram(X.numpy(), plan.split_rows, True, s=s)
    assert_bits(G, Go, "G (scaled)")
    assert_bits(npart, npo, "norm partials (scaled)")


@pytest.mark.parametrize("K,r", SHAPES + SHAPES32 + SHAPESW)
@pytest.mark.parametrize("name", ["mixed_c4", "rank_half", "zero"])
def test_chol(cuda, K, r, name):
    print(f"chol {K}x{r} {name}", flush=True)
    X = case_x(K, r, name)
    plan = get_plan(K, r, cuda)
    Go, npo = oracle.gram(X.numpy(), plan.split_rows, True)
    L, Li, sc = stages.chol(torch.from_numpy(Go).to(cuda), torch.from_numpy(npo).to(cuda), K)
    nrm = oracle.norm(npo)
    Gs, tau = oracle.shift(Go, nrm)
    Lo, Lio = oracle.chol(Gs, tau)
    sc = sc.cpu().numpy()
    assert sc[2] == 0, "grid barrier timed out"
    assert_bits(sc[:2], np.array([nrm, tau], np.float32), "nrm, tau")
    assert_bits(torch.tril(L), Lo, "L")
    assert_bits(Li, Lio, "Li")


@pytest.mark.parametrize("K,r", SHAPES)
def test_chol32_absolute(cuda, K, r):
    print(f"chol32 {K}x{r}", flush=True)
    X = case_x(K, r, "mixed_c8")
    G = X.double().T @ X.double()
    G = (G + 1e-7 * torch.linalg.matrix_norm(G) * torch.eye(r, dtype=torch.float64)).float().numpy()
    tau = np.float32(1e-6)
    L, Li = stages.chol32(torch.from_numpy(G).to(cuda), float(tau), K)
    Lo, Lio = oracle.chol(G, tau)
    assert_bits(torch.tril(L), Lo, "L")
    assert_bits(Li, Lio, "Li")


# K >= 9216 (r <= 256) takes the row-blocked solve (a wavefront pair per 16 rows), below it the column-blocked one
# (16400 x 384: two column blocks per wave and two row blocks per workgroup, the last one past K); ragged K on all
@pytest.mark.parametrize("K,r", SHAPES + [(16384, 256), (32768, 64), (4100, 128), (4111, 192), (9230, 192),
                                          (16400, 256), (16425, 128), (16400, 384)] + SHAPES32 +
                         [(9300, 96), (10000, 224), (16400, 288)] + SHAPESW + [(9000, 800)])
@pytest.mark.parametrize("pass1", [True, False])
def test_trsm(cuda, K, r, pass1):
    print(f"trsm {K}x{r} pass1={pass1}", flush=True)
    X = case_x(K, r, "ttf_cu4_t1e-2")
    plan = get_plan(K, r, cuda)
    Xn = X.numpy()
    s = oracle.pow2_scale(oracle.amax(Xn))
    Go, npo = oracle.gram(Xn, plan.split_rows, True, s=s)
    Gs, tau = oracle.shift(Go, oracle.norm(npo))
    Lo, Lio = oracle.chol(Gs, tau)
    Xd = X.to(cuda)
    if pass1:
        stages.amax(Xd)
    Y = stages.trsm(Xd, torch.from_numpy(Lo).to(cuda), torch.from_numpy(Lio).to(cuda), pass1=pass1)
    if pass1:
        Yo = oracle.trsm(Xn, Lo, Lio, s=s, Z=oracle.dust(K, r), eps=5e-7)
    else:
        Yo = oracle.trsm(Xn, Lo, Lio)
    assert_bits(Y, Yo, "Y")


# grids of at most two workgroups per CU take the two-buffer Newton-Schulz apply: ragged K, 64-column steps
# (r % 128 == 0) and 32-column steps (r % 128 == 64), an even number of them
SHAPES_NSP = [(1000, 384), (777, 320), (2100, 448)]
# more than two workgroups per CU and r <= 512 take the apply with D's columns held in registers: 16-row blocks,
# ragged K, one to eight 64-column slabs (r <= 256 and r <= 512 forms)
SHAPES_NSR = [(17408, 256), (9000, 128), (6001, 192), (20000, 64), (4100, 512), (5000, 320)]


@pytest.mark.parametrize("K,r", SHAPES + SHAPES32 + SHAPESW + SHAPES_NSP + SHAPES_NSR)
@pytest.mark.parametrize("kahan", [True, False])
def test_ns_step(cuda, K, r, kahan):
    print(f"ns {K}x{r} kahan={kahan}", flush=True)
    X = case_x(K, r, "mixed_c2")
    Y = (torch.linalg.qr(X.double())[0].float() * 1.0001).contiguous()
    plan = get_plan(K, r, cuda)
    out = stages.ns_step(Y.to(cuda), kahan)
    Go, _ = oracle.gram(Y.numpy(), plan.split_rows, kahan)
    Yo = oracle.ns_apply(Y.numpy(), oracle.ns_D(Go))
    assert_bits(out, Yo, "NS step")


ORTH_CASES = [(256, 64, "mixed_c4"), (256, 128, "zero"), (384, 256, "rank_half"), (768, 512, "ttf_cu4_t1e-2"),
              (768, 512, "dup_cols"), (1024, 256, "huge_1e25"), (1024, 256, "tiny_1e-25"), (2048, 512, "mixed_c8"),
              (17408, 256, "ttf_cu4_t1e-2"), (4100, 192, "mixed_c6"),
              (64, 32, "zero"), (300, 96, "mixed_c4"), (1000, 160, "rank_half"), (4100, 224, "ttf_cu4_t1e-2"),
              (768, 480, "mixed_c8"), (12000, 160, "mixed_c4"), (2048, 352, "huge_1e25"),
              (600, 544, "mixed_c4"), (2000, 800, "ttf_cu4_t1e-2"), (1024, 992, "rank_half"), (4096, 640, "huge_1e25"),
              (672, 672, "zero")]


@pytest.mark.parametrize("K,r,name", ORTH_CASES)
def test_orth_bit_exact(cuda, K, r, name):
    print(f"orth {K}x{r} {name}", flush=True)
    X = case_x(K, r, name)
    Xd = X.to(cuda)
    X0 = Xd.clone()
    Q1 = orth(Xd)
    Q2 = orth(Xd)
    torch.cuda.synchronize()
    assert_bits(Q1, Q2, "repeat")
    assert_bits(Xd, X0, "input intact")
    plan = get_plan(K, r, cuda)
    assert stages.scalars(K, r, cuda)[7].item() == 0, "grid barrier timed out"
    Qo = oracle.orth(X.numpy(), plan.split_rows)
    assert_bits(Q1, Qo, "Q")
