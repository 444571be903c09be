"""The reference's benchmark runner (src/benchmark/), for this library's configs.

``python -m cernels_amd.benchmark.main <config>`` times a config's workloads the way the reference's
``python -m benchmark.main <config>`` does and writes ``analysis/<host>/<config>.{json,log}``;
``python -m cernels_amd.benchmark.view`` prints the saved records as one table. Everything runs
offline: there is no Hub, so a config whose reference is a Hub kernel times its ``custom`` workload
alone.
"""
