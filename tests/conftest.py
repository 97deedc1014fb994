import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "drama3-mlx_amd"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import d3s_oracle
    d3s_oracle.lib()
    return d3s_oracle


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Rows, id mismatches and boundary rows of every configuration the GPU
    parity tests compared (BASELINE.json's C1-C5 first)."""
    try:
        import parity_report
    except ImportError:
        return
    recs = parity_report.RECORDS
    if not recs:
        return
    tr = terminalreporter
    tr.section("parity: rows / id mismatches / boundary rows")
    configs = [r for r in recs if r[0].startswith("config ")]
    for label, rows, bad, edge in configs:
        tr.write_line(f"{label}: rows {rows}, id mismatches {bad}, boundary rows {edge}")
    tot = [sum(r[i] for r in recs) for i in (1, 2, 3)]
    tr.write_line(f"all {len(recs)} comparisons: rows {tot[0]}, id mismatches {tot[1]}, "
                  f"boundary rows {tot[2]}")
