"""Seeded workload generators shared by the benchmark, the tests and the promotion evaluation."""
