"""The CPU oracle is pinned to the reference's algorithm (tests/pins.py), and the pins have teeth: a copy of the
oracle with any one planted defect (oracle/kcholf_oracle.c, PLANTED(n)) fails at least one of them."""
import pytest

import oracle
import pins

DEFECTS = {
    1: "trailing update with the wrong sign",
    2: "tile inverse scaled by the wrong pivot reciprocal",
    3: "panel multiplied by Li instead of Li^T",
    4: "solve reads L transposed",
    5: "Newton-Schulz correction without the 1/2",
    6: "Kahan compensation with the wrong sign",
    7: "diagonal shift dropped",
    8: "pivot clamp with fminf instead of fmaxf",
    9: "dust columns not normalised",
    10: "power-of-2 scale rounds up instead of to nearest",
    11: "block projection product reads the wrong column of C",
    12: "block projection adds P P^T C instead of subtracting it",
    13: "every block gets the first dust slice",
    14: "blocks projected once before orthonormalisation instead of twice",
    15: "fp64 trailing update with the wrong sign",
    16: "max|x| as a signed maximum (absolute value dropped)",
}


@pytest.mark.parametrize("check", pins.ALL, ids=lambda c: c.__name__)
def test_oracle_pinned(check):
    assert check() == []


@pytest.fixture(scope="module")
def plant_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("planted")


@pytest.mark.parametrize("n", sorted(DEFECTS), ids=lambda n: f"{n}-{DEFECTS[n].replace(' ', '_')}")
def test_planted_defect_is_caught(n, plant_dir):
    with oracle.planted(n, plant_dir):
        caught = {c.__name__: c() for c in pins.ALL}
    assert any(caught.values()), f"planted defect {n} ({DEFECTS[n]}) passes every check"
