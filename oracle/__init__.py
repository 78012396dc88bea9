"""CPU oracle for the compressed-KV decode hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from this package, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement).  The product path
(``rina-1bit-kv_amd/modules`` + ``libkvr_hip.so``) never imports it and has no
CPU fallback: without the HIP library it raises.

Modules
-------
kvr_oracle : numpy restatement of every kernel of the path (transform, tile
             scale, sigma-delta, packing, tile scoring, top-k, decode
             attention), emulating the kernels' fp32 operation order where the
             contract is bit-exact and computing in float64 where it is a
             tolerance.

Pinning status of each oracle function is listed in ``kvr_oracle.__doc__``.
"""
