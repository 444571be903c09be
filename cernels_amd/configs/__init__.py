"""Workload configurations: the benchmark shapes, seeded synthetic inputs, routers."""
