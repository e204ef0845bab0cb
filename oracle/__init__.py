"""TEST INFRASTRUCTURE — the CPU oracle for the IRON decode/prefill operator path.

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
bench.py may import this package, and only as the checker (or the timed CPU
baseline). The library (iron_amd/) never imports it and has no CPU fallback.

Contents
  ops.py      torch/numpy restatements of each reference operator's
              ``reference()`` and seeded golden generator, citing the
              reference file:line each follows.
  configs.py  the BASELINE.json configurations as seeded synthetic inputs.
  llama.py    restatement of the fp32 CPU Llama forward
              (iron/applications/llama_3.2_1b/llama_cpu.py).

Pinning (what checks each function; tests/test_oracle_*.py): see the
``PINNED BY`` line in each docstring. A function whose line says
"parity unpinned" has no independent check.

The reference itself is Python that imports absent packages (mlir_aie,
ml_dtypes, tiktoken); it is read as text and never imported or run here, and
it ships no C/C++ source, so there is no oracle/_ref build.
"""
