"""CPU oracle for the compressed-KV attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of bhengubv/shard's
compressed-KV path (``src/shard/{cache,attention,rope,streaming,triton_kernels}.py``)
so that the HIP implementation in ``shard_amd`` can be checked against it.

Rules for use:
  * Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
    ``bench.py`` may import anything under ``oracle/``, and only as the checker
    (or the timed CPU baseline), never as the product path.
  * ``shard_amd`` never imports this package; the product fails loudly when its
    HIP library is missing instead of falling back here.

Modules:
  ``ref``    — op-for-op restatement of the reference PyTorch CPU fallback path
               (fp16 cast points kept), numpy for the bit-exact integer chains.
  ``exact``  — fp64 evaluation of attention over the dequantized representation
               (the accuracy yardstick for attention outputs).
  ``synth``  — seeded synthetic inputs of the benchmark workloads (Llama-3.1-8B
               attention-layer shapes).

Parity-pinning status of every function is listed in each module's header.
"""
