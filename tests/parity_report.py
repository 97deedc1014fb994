"""Per-configuration parity counts collected by the GPU parity tests and printed
in pytest's terminal summary (tests/conftest.py), so that boundary rows are
counted and reported even under -q.  A boundary row is one whose float64 shadow
puts a cumulative value within 1e-6 of top_p or the top two race scores within
1e-6 relative (oracle flags TOPP_EDGE / RACE_EDGE): an fp32 implementation with
another summation order could sample another id there."""

RECORDS = []


def record(label, rows, mismatched, boundary):
    RECORDS.append((label, int(rows), int(mismatched), int(boundary)))
