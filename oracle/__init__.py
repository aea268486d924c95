"""CPU oracle for the DRAFTKV decode round -- TEST INFRASTRUCTURE ONLY.

This package is a numpy restatement of the reference algorithm (aabhimittal/
Draft-KV, pure Python + numpy) for the self-speculative decode round: group
quantization, the compressed drafter mirror with sink/recent/heavy-hitter
eviction, the paged full cache with its LIFO block pool, masked softmax
attention, the sampling helpers and the draft -> verify -> accept -> resync
loop, and the three model forwards that drive it.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.
The product package (``draftkv`` under ``draft-kv_amd/``) never imports it and
has no CPU fallback: every product computation runs in the HIP library.

Each function cites the reference file:line whose behaviour it restates. The
numpy version followed is 2.2 (NEP 50 promotion rules: a float32 array divided
by ``np.sqrt(int)`` -- a float64 numpy scalar -- becomes float64; divided by a
Python int it stays float32).
"""
