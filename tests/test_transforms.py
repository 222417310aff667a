"""polyattn.transforms.kv_per_tile of the drop-in package, pinned by the reference's own
recorded values (tests/test_transforms.py:20-25 and tests/test_findings.py:60-74,157-168
of the reference) and by brute force over the offset set."""
import itertools
import sys

import pytest

from tests.conftest import ROOT

sys.path.insert(0, str(ROOT / "polyhedral_amd"))
from polyattn import transforms  # noqa: E402  (the bare-name import a driver makes)


def test_reference_recorded_values():
    assert transforms.kv_per_tile("A", 0, 1, 16, 16) == 16
    assert transforms.kv_per_tile("B", 1, 1, 16, 16) == 16 + 15
    assert transforms.kv_per_tile("B", 1, 8, 16, 16) == 136
    # the lower / upper bracket of class B (BQ * A rows without sharing) at three tiles
    for BQ, A, gap in ((128, 128, 64.3), (128, 32, 25.8), (16, 16, 8.3)):
        lo = transforms.kv_per_tile("B", 1, 1, BQ, A)
        assert BQ * A / lo == pytest.approx(gap, rel=0.02)
        assert lo > transforms.kv_per_tile("A", 0, 1, BQ, A)


@pytest.mark.parametrize("a,s,BQ,A", [(1, 1, 128, 32), (2, 3, 16, 16), (0, 4, 8, 16), (3, 0, 16, 8),
                                      (4, 2, 32, 16), (1, 16, 16, 16), (5, 7, 8, 8)])
def test_class_b_equals_brute_force(a, s, BQ, A):
    want = len({a * x - s * y for x, y in itertools.product(range(BQ), range(A))})
    assert transforms.kv_per_tile("B", a, s, BQ, A) == want


def test_closed_forms_and_errors():
    # unit shear: A + BQ - 1 rows; no shear: the A columns; no stride: the BQ offsets
    assert transforms.kv_per_tile("B", 1, 1, 128, 32) == 159
    assert transforms.kv_per_tile("B", 0, 3, 64, 16) == 16
    assert transforms.kv_per_tile("B", 2, 0, 64, 16) == 64
    with pytest.raises(ValueError):
        transforms.kv_per_tile("C", 1, 1, 16, 16)
