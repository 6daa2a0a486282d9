"""bench.py's measurement plumbing on the CPU: every leg's roofline class finds its HBM traffic
in the committed PMC summaries, and the figure is per launch of that class (not a whole run)."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    sys.path.insert(0, REPO)
    import bench as b

    return b


@pytest.mark.parametrize("kernel,leg,algorithmic", [
    ("enc_chain", "", 1157627904),    # 80 ms headline: the 24 blocks' weights read once per launch
    ("gemm_fr*", "S560", 7400220),
    ("gemm_fr*", "S1120", 6242544),
    ("gemm_m*", "B64", None),
    ("gemm_m*", "B256", None),
])
def test_traffic_marker_per_leg(bench, kernel, leg, algorithmic):
    t = bench.traffic_from_profile(kernel, leg)
    assert t is not None, (kernel, leg)
    if algorithmic:
        # a weight-streaming class cannot move fewer bytes than its weights, and re-reads stay bounded
        assert algorithmic <= t < 2 * algorithmic
    else:
        # many-row GEMMs: tens to hundreds of MB per launch at 448 / 3584 rows
        assert 5e6 < t < 1e9


def test_traffic_marker_unknown_class(bench):
    assert bench.traffic_from_profile("no_such_kernel*", "S560") is None
