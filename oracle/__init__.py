"""CPU oracle for the packed-attention hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product path (``minifield-training_amd/``) imports, links or
executes anything in this package.  Only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker
or as the timed CPU baseline, never as the thing being measured on the GPU.

Modules
-------
``packing``   restatement of the reference row packer (first-fit decreasing)
              and of the seeded BASELINE workload generators.
``masks``     validity grids and the brute-force tile-map reduction.
``attention`` FP64 masked-softmax attention, its analytic VJP, the cached
              decode oracle and torch-CPU emulations of the reference's bf16
              cast points.
``workload``  useful-pair, FLOP and byte accounting.

Parity pinning (what each function is checked against) is listed in each
module docstring; ``tests/test_oracle_*.py`` hold the checks.
"""
