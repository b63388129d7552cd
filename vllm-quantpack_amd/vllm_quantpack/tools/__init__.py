"""Benchmark and test helpers: seeded synthetic paged caches."""
