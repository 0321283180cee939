"""Workload parameters shared by tests/golden/make_golden.py and the tests."""
PREFILL_LENS = [1, 17, 64, 90]
PREFILL_HEADS = (4, 2)
